"""trnblas_amd — the Level-3 hot path of trnsci/trnblas on AMD MI355X.

A drop-in for `trnblas`'s Level-3 API on PyTorch-ROCm (`import trnblas_amd
as trnblas`): `gemm`, `batched_gemm`, `syrk`, `gemm_fp64`, `trsm`,
`metric_inv_half`, the DF-MP2 pair
energy (`hip.nki_batched_pair_energy`), the backend switches and the
`torch.ops.trnblas.*` op surface (`hip.get_native_ops()`). Device operands
run hand-written gfx950 kernels from `libtrnblas_hip.so` (C ABI:
include/trnblas_hip.h); the host half is Python.
"""

__version__ = "0.1.0"

from . import hip  # noqa: F401
from . import ozaki  # noqa: F401
from .hip import get_autotune, get_backend, get_cores, set_autotune, set_backend, set_cores
from .level3 import batched_gemm, gemm, gemm_fp64, metric_inv_half, syrk, trsm

nki = hip  # the reference's subpackage name


def __getattr__(name):
    if name in ("HAS_HIP", "HAS_NKI"):
        return hip.has_hip()
    raise AttributeError(name)


__all__ = [
    "gemm",
    "gemm_fp64",
    "batched_gemm",
    "syrk",
    "trsm",
    "metric_inv_half",
    "HAS_HIP",
    "HAS_NKI",
    "set_backend",
    "get_backend",
    "set_autotune",
    "get_autotune",
    "set_cores",
    "get_cores",
]
