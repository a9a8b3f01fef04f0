"""ctypes binding of libtheria_sdpa.so (the C ABI declared in include/theria_sdpa.h).

The library is loaded lazily, after torch, so that it binds to the HIP runtime torch already loaded
(both carry the soname libamdhip64.so.7). There is no fallback: if the library is missing or was
built for another ABI version, loading raises, and every HIP-backed operator fails loudly.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch  # noqa: F401  (must be imported first: it loads the HIP runtime the library binds to)

# The in-tree build (the torch binding _theria_host is linked against this same file).
LIB_PATH = Path(__file__).resolve().parent / "lib" / "libtheria_sdpa.so"
# The counter-enabled build of the same sources (theria_debug_tile_counts counts there), for measurements only.
TILES_LIB_PATH = LIB_PATH.with_name("libtheria_sdpa_tiles.so")
ABI_VERSION = 9

DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
OK, ERR_CONTRACT, ERR_HIP = 0, 1, 2

# Every symbol the header declares, with its ctypes signature.
_P = ctypes.c_void_p


class TensorView(ctypes.Structure):
    """theria_tensor_t: (B, H, rows, D) view with element strides; last dim contiguous."""

    _fields_ = [
        ("data", ctypes.c_void_p),
        ("stride_b", ctypes.c_int64),
        ("stride_h", ctypes.c_int64),
        ("stride_row", ctypes.c_int64),
    ]


class Problem(ctypes.Structure):
    """theria_sdpa_problem_t."""

    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("tq", ctypes.c_int32),
        ("tk", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("causal", ctypes.c_int32),
    ]


_TV = ctypes.POINTER(TensorView)
_PR = ctypes.POINTER(Problem)
_FP = ctypes.POINTER(ctypes.c_float)

SIGNATURES = {
    "theria_abi_version": ([], ctypes.c_int),
    "theria_last_error": ([], ctypes.c_char_p),
    "theria_sdpa_fwd": ([_PR, _TV, _TV, _TV, _TV, ctypes.c_int32, _P, _P, _P, _P], ctypes.c_int),
    "theria_sdpa_bwd": (
        [_PR, _TV, _TV, _TV, _TV, ctypes.c_int32, _TV, _P, _P, _TV, _TV, _TV, _P],
        ctypes.c_int,
    ),
    "theria_sdpa_bwd_dq": ([_PR, _TV, _TV, _TV, _TV, ctypes.c_int32, _TV, _P, _P, _TV, _P], ctypes.c_int),
    "theria_sdpa_bwd_dkdv": ([_PR, _TV, _TV, _TV, _TV, _P, _P, _TV, _TV, _P], ctypes.c_int),
    "theria_sdpa_bwd_from_stats": (
        [_PR, _TV, _TV, _TV, _TV, _P, _P, _TV, _TV, _TV, ctypes.c_int32, _P],
        ctypes.c_int,
    ),
    "theria_sdpa_jvp": ([_PR, _TV, _TV, _TV, _TV, _P, _TV, _TV, _TV, _TV, ctypes.c_int32, _P], ctypes.c_int),
    "theria_sdpa_bwd_bwd": (
        [_PR, _TV, _TV, _TV, _TV, _TV, _P, _P, _TV, _TV, _TV, _TV, _TV, _TV, _TV, _P, _P],
        ctypes.c_int,
    ),
    "theria_sdpa_bwd_bwd_noalloc": (
        [_PR, _TV, _TV, _TV, _TV, _TV, _P, _P, _TV, _TV, _TV, _TV, _TV, _TV, _TV, _P],
        ctypes.c_int,
    ),
    "theria_qk_scores": ([_PR, _TV, _TV, _P, ctypes.c_int32, _P], ctypes.c_int),
    "theria_qk_softmax": ([_PR, _TV, _TV, _P, _P], ctypes.c_int),
    "theria_debug_tile_counts": ([ctypes.POINTER(ctypes.c_uint64), ctypes.c_int32], ctypes.c_int),
    "theria_debug_atomic_probe": ([_P, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, _P], ctypes.c_int),
}

_lock = threading.Lock()
_lib = None


class TheriaError(RuntimeError):
    """A HIP launch failure reported by libtheria_sdpa.so."""


def load(path: str | os.PathLike | None = None):
    """Load (once) and return the ctypes library handle; raise if it is missing or incompatible."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise RuntimeError(
                f"theria_amd: {p} is not built. Run `python -m theria_amd.build` (needs hipcc) before "
                "using the HIP SDPA operators; there is no fallback path."
            )
        lib = ctypes.CDLL(str(p), mode=ctypes.RTLD_LOCAL)
        for name, (argtypes, restype) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = restype
        ver = lib.theria_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"theria_amd: library ABI {ver} != expected {ABI_VERSION}; rebuild it")
        if path is None:
            _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    """Map a C status to the reference's error conventions (AssertionError for contract violations)."""
    if rc == OK:
        return
    msg = (load().theria_last_error() or b"").decode(errors="replace")
    if rc == ERR_CONTRACT:
        raise AssertionError(f"{what}: {msg}")
    raise TheriaError(f"{what}: {msg}")
