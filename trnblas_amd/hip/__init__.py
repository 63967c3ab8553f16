"""HIP (gfx950) dispatch of trnblas_amd — the counterpart of `trnblas.nki`.

Exports the reference's `trnblas.nki` names (trnblas/nki/__init__.py:3-36),
so `from trnblas_amd.hip import nki_batched_pair_energy` works as
`from trnblas.nki import nki_batched_pair_energy` did. Importing this
package loads no native library and registers no op.
"""

from .dispatch import (
    HipFallbackWarning,
    NkiFallbackWarning,
    get_autotune,
    get_backend,
    get_native_ops,
    has_hip,
    nki_batched_gemm,
    nki_batched_pair_energy,
    nki_fused_gemm_energy,
    nki_gemm,
    nki_gemm_fp64,
    nki_mp2_energy,
    nki_metric_inv_half,
    nki_syrk,
    nki_trsm,
    set_autotune,
    set_backend,
)

_cores = 1


def set_cores(n: int) -> None:
    """One MI355X per process: only 1 is accepted (the reference's multi-core
    split, trnblas/nki/multicore.py, is out of scope on one GPU)."""
    if int(n) != 1:
        raise ValueError("trnblas_amd runs one GPU per process: set_cores(1) only")


def get_cores() -> int:
    return _cores


def __getattr__(name):
    if name in ("HAS_HIP", "HAS_NKI"):
        return has_hip()
    raise AttributeError(name)


__all__ = [
    "HAS_HIP",
    "HAS_NKI",
    "HipFallbackWarning",
    "NkiFallbackWarning",
    "set_backend",
    "get_backend",
    "set_autotune",
    "get_autotune",
    "set_cores",
    "get_cores",
    "get_native_ops",
    "nki_gemm",
    "nki_batched_gemm",
    "nki_batched_pair_energy",
    "nki_fused_gemm_energy",
    "nki_gemm_fp64",
    "nki_mp2_energy",
    "nki_syrk",
    "nki_trsm",
    "nki_metric_inv_half",
]
