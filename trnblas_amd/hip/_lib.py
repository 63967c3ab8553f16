"""ctypes binding of `libtrnblas_hip.so` (the C ABI in include/trnblas_hip.h).

The library is loaded lazily on first use, after torch (whose bundled HIP
runtime then also serves the library: both resolve `libamdhip64.so.7`, so
streams and device pointers are shared). There is no fallback: a missing or
unloadable library raises `HipLibraryError`, and callers that asked for the
HIP path see that error.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch  # noqa: F401  (loads torch's HIP runtime before the library)

_PKG = Path(__file__).resolve().parent.parent
LIB_PATH = Path(os.environ.get("TRNBLAS_HIP_LIB", _PKG / "lib" / "libtrnblas_hip.so"))

ABI_VERSION = 11

F32, BF16, F16, F64 = 0, 1, 2, 3
DTYPE_CODES = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}

# bits of trnblas_hip_dgemm's `tri`
TRI_A_LOWER, TRI_A_UPPER, TRI_B_LOWER, TRI_B_UPPER = 1, 2, 4, 8

E_ARG, E_LAUNCH, E_NONFINITE, E_WORKSPACE = -1, -2, -3, -4

_c_i64 = ctypes.c_int64
_c_int = ctypes.c_int
_c_dbl = ctypes.c_double
_c_ptr = ctypes.c_void_p
_c_size = ctypes.c_size_t

# name -> (restype, argtypes); the exported surface of include/trnblas_hip.h
SIGNATURES = {
    "trnblas_hip_abi_version": (_c_int, []),
    "trnblas_hip_last_error": (ctypes.c_char_p, []),
    "trnblas_hip_gemm": (
        _c_int,
        [_c_int, _c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_dbl]
        + [_c_ptr, _c_i64, _c_i64] * 2
        + [_c_dbl, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr, _c_size]
        + [_c_ptr],
    ),
    "trnblas_hip_gemm_workspace": (_c_size, []),
    "trnblas_hip_pack_k": (
        _c_int,
        [_c_int, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64]
        + [_c_ptr],
    ),
    "trnblas_hip_syrk": (
        _c_int,
        [_c_int, _c_int, _c_int, _c_i64, _c_i64, _c_dbl, _c_ptr, _c_i64, _c_dbl, _c_ptr]
        + [_c_i64, _c_ptr, _c_i64, _c_ptr, _c_size, _c_ptr],
    ),
    "trnblas_hip_syrk_flagged": (
        _c_int,
        [_c_int, _c_int, _c_int, _c_i64, _c_i64, _c_dbl, _c_ptr, _c_i64, _c_dbl, _c_ptr]
        + [_c_i64, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_size, _c_ptr],
    ),
    "trnblas_hip_triangle_nonzero": (_c_int, [_c_int, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_ptr]),
    "trnblas_hip_pair_energy_workspace": (_c_size, [_c_i64, _c_i64]),
    "trnblas_hip_pair_energy": (
        _c_int,
        [_c_i64, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr]
        + [_c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_size, _c_ptr],
    ),
    "trnblas_hip_pair_energy_bf16x6_workspace": (_c_size, [_c_i64] * 5),
    "trnblas_hip_pair_energy_bf16x6": (
        _c_int,
        [_c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64]
        + [_c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr]
        + [_c_ptr, _c_size, _c_ptr],
    ),
    "trnblas_hip_pair_energy_fp16x3_workspace": (_c_size, [_c_i64] * 5),
    "trnblas_hip_pair_energy_fp16x3": (
        _c_int,
        [_c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64]
        + [_c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr]
        + [_c_ptr, _c_size, _c_ptr],
    ),
    "trnblas_hip_pair_energy_noalloc_max_bytes": (_c_size, []),
    "trnblas_hip_pair_energy_noalloc": (
        _c_int,
        [_c_i64, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr]
        + [_c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr],
    ),
    "trnblas_hip_mp2_energy": (
        _c_int,
        [_c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr],
    ),
    "trnblas_hip_ozaki_split": (
        _c_int,
        [_c_int, _c_i64, _c_i64, _c_ptr, _c_i64, _c_int, _c_ptr, _c_i64, _c_i64, _c_ptr]
        + [_c_ptr, _c_ptr],
    ),
    "trnblas_hip_ozaki_gemm": (
        _c_int,
        [_c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_ptr]
        + [_c_i64, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64, _c_ptr],
    ),
    "trnblas_hip_ozaki_hilo": (
        _c_int,
        [_c_int, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64]
        + [_c_ptr, _c_i64, _c_ptr],
    ),
    "trnblas_hip_crt_moduli": (_c_int, [_c_int, _c_i64]),
    "trnblas_hip_crt_split": (
        _c_int,
        [_c_int, _c_i64, _c_i64, _c_ptr, _c_i64, _c_int, _c_int, _c_i64, _c_ptr, _c_i64]
        + [_c_ptr, _c_ptr, _c_ptr],
    ),
    "trnblas_hip_crt_gemm": (
        _c_int,
        [_c_int, _c_i64, _c_i64, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr],
    ),
    "trnblas_hip_crt_combine": (
        _c_int,
        [_c_int, _c_int, _c_i64, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_ptr, _c_i64, _c_i64]
        + [_c_ptr],
    ),
    "trnblas_hip_chol_block": (
        _c_int,
        [_c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr],
    ),
    "trnblas_hip_tri_inv_blocks": (
        _c_int,
        [_c_int, _c_i64, _c_int, _c_int, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_ptr],
    ),
    "trnblas_hip_metric_inv_half_workspace": (_c_size, [_c_i64]),
    "trnblas_hip_metric_inv_half": (
        _c_int,
        [_c_i64, _c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr, _c_ptr, _c_size, _c_ptr],
    ),
    "trnblas_hip_trsm_workspace": (_c_size, [_c_int, _c_i64, _c_i64]),
    "trnblas_hip_trsm": (
        _c_int,
        [_c_int, _c_i64, _c_i64, _c_int, _c_int, _c_dbl]
        + [_c_ptr, _c_i64, _c_i64] * 3
        + [_c_ptr, _c_size, _c_ptr],
    ),
    "trnblas_hip_dgemm": (
        _c_int,
        [_c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_dbl]
        + [_c_ptr, _c_i64, _c_i64] * 2
        + [_c_dbl, _c_ptr, _c_i64, _c_i64, _c_ptr, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _c_ptr],
    ),
}


class HipLibraryError(RuntimeError):
    """The HIP op library is missing, stale, or cannot be loaded."""


class HipKernelError(RuntimeError):
    """A C-ABI call returned an error code."""

    def __init__(self, fn: str, code: int, message: str):
        super().__init__(f"{fn} failed ({code}): {message}")
        self.fn, self.code, self.message = fn, code, message


_lib = None
_lock = threading.Lock()


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """The loaded library (cached). Raises HipLibraryError if it cannot be loaded."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise HipLibraryError(
                f"{p} not found: build it with `python -m trnblas_amd.build` "
                "(or __graft_entry__.build())"
            )
        try:
            lib = ctypes.CDLL(str(p))
        except OSError as exc:
            raise HipLibraryError(f"cannot load {p}: {exc}") from exc
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name, None)
            if fn is None:
                continue  # reported by missing_symbols(); calling it raises
            fn.restype = res
            fn.argtypes = args
        v = lib.trnblas_hip_abi_version()
        if v != ABI_VERSION:
            raise HipLibraryError(f"{p}: ABI version {v}, expected {ABI_VERSION} (rebuild)")
        if path is None:
            _lib = lib
        return lib


def missing_symbols(lib: ctypes.CDLL | None = None) -> list[str]:
    """Entry points of include/trnblas_hip.h the loaded library lacks."""
    lib = lib or load()
    return [n for n in SIGNATURES if getattr(lib, n, None) is None]


def available() -> bool:
    try:
        load()
        return True
    except HipLibraryError:
        return False


def call(name: str, *args) -> int:
    """Call C-ABI function `name`; raise HipKernelError on a negative return."""
    lib = load()
    fn = getattr(lib, name, None)
    if fn is None:
        raise HipLibraryError(f"{LIB_PATH} does not export {name} (rebuild)")
    rc = fn(*args)
    if rc < 0:
        msg = lib.trnblas_hip_last_error()
        raise HipKernelError(name, rc, msg.decode() if msg else "")
    return rc


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    """hipStream_t of torch's current stream on `device`, as an int (the raw
    lookup: torch.cuda.current_stream builds a Stream object per call, a few
    microseconds on every launch)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(idx)


def broadcast_shapes(a, b) -> tuple:
    """torch.broadcast_shapes for two shapes, in plain Python (torch's goes
    through its symbolic-shape machinery, ~10 us per call on the launch
    path); the same RuntimeError on shapes that do not broadcast."""
    a, b = tuple(a), tuple(b)
    n = max(len(a), len(b))
    a = (1,) * (n - len(a)) + a
    b = (1,) * (n - len(b)) + b
    out = []
    for x, y in zip(a, b):
        if x == y or y == 1:
            out.append(x)
        elif x == 1:
            out.append(y)
        else:
            raise RuntimeError(f"shapes {a} and {b} are not broadcastable")
    return tuple(out)
