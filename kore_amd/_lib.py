"""ctypes binding of libkore_amd.so (the C ABI declared in include/kore_amd.h).

The library is loaded from this package directory only.  There is no fallback: if
the shared library is missing or a symbol is absent, every operator raises.
"""

from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libkore_amd.so"

KORE_OK = 0
_ERRORS = {1: ValueError, 2: NotImplementedError, 3: RuntimeError, 4: ValueError}

_vp, _i64, _i32, _sz = C.c_void_p, C.c_int64, C.c_int, C.c_size_t

# name -> (restype, argtypes); mirrors include/kore_amd.h exactly.
SIGNATURES = {
    "kore_last_error": (C.c_char_p, []),
    "kore_abi_version": (_i32, []),
    "kore_gemm_workspace_bytes": (_sz, [_i32, _i32, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _i64,
                                        _i64, _i64, _i64]),
    "kore_gemm": (_i32, [_i32, _i32, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _i64,
                         _i64, _i64, _i64, _vp, _sz, _vp]),
    "kore_gemm_noalloc_scratch_bytes": (_sz, []),
    "kore_gemm_noalloc": (_i32, [_i32, _i32, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _i64,
                                 _i64, _i64, _i64, _vp]),
    "kore_batched_gemm_workspace_bytes": (_sz, [_i32, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64,
                                                _vp, _i64, _i64, _i64, _i64, _i64, _i64]),
    "kore_batched_gemm": (_i32, [_i32, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64,
                                 _vp, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _sz, _vp]),
    "kore_gemm_backward_workspace_bytes": (_sz, [_i32, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64,
                                                 _i64, _i64, _i64]),
    "kore_gemm_backward": (_i32, [_i32, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i64,
                                  _vp, _sz, _vp]),
    "kore_gemm_a8w8_blockscale": (_i32, [_vp, _i64, _vp, _i64, _vp, _i64, _i64, _vp, _i64,
                                         _i64, _vp, _i64, _i64, _i64, _i64, _vp]),
    "kore_gemm_a8w8": (_i32, [_i32, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _i64, _vp, _i64,
                              _i64, _i64, _i64, _vp]),
    "kore_moe_align_capacity": (_i64, [_i64, _i64, _i64, _i64]),
    "kore_moe_test_force_generic": (_i32, [_i32]),
    "kore_moe_grouped_gemm_workspace_bytes": (_sz, [_i64, _i64]),
    "kore_moe_grouped_gemm": (_i32, [_vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _sz, _vp]),
    "kore_moe_grouped_gemm_fp8": (_i32, [_vp, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                         _vp, _sz, _vp]),
    "kore_gather_rows": (_i32, [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _vp]),
    "kore_scatter_rows": (_i32, [_vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _vp]),
    "kore_moe_align": (_i32, [_vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _vp]),
    "kore_fused_moe_workspace_bytes": (_sz, [_i64, _i64, _i64, _i64, _i64]),
    "kore_fused_moe": (_i32, [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64,
                              _i64, _vp, _sz, _vp]),
}

_lock = threading.Lock()
_lib = None


def load() -> C.CDLL:
    """Load (once) and return the library with every signature bound."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is not built; run `python kore_amd/build.py` "
                    "(hipcc --offload-arch=gfx950). kore_amd has no non-HIP fallback.")
            lib = C.CDLL(str(LIB_PATH))
            missing = [n for n in SIGNATURES if not hasattr(lib, n)]
            if missing:
                raise RuntimeError(f"{LIB_PATH} lacks exported symbols {missing}; rebuild it")
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(rc: int) -> None:
    """Raise the Python exception matching a non-zero C-ABI status."""
    if rc == KORE_OK:
        return
    msg = load().kore_last_error().decode(errors="replace")
    raise _ERRORS.get(rc, RuntimeError)(f"kore_amd error {rc}: {msg}")
