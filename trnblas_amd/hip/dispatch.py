"""HIP dispatch of trnblas_amd: backend selection, routing, dtype policy.

The MI355X counterpart of trnblas/nki/dispatch.py (host half, :1-3310).
What stays: the public entry points (`nki_gemm`, `nki_batched_gemm`,
`nki_syrk`, `nki_batched_pair_energy`, `nki_fused_gemm_energy`,
`nki_mp2_energy`, `nki_gemm_fp64`), the backends `auto` / `pytorch` plus the
kernel backend (`hip`, with `nki` accepted as its alias), the route names of
`_gemm_route` (:633-682), the kernel-dtype backstop (`_check_kernel_operands`,
:1244-1293), the result-dtype rules (:1328-1340) and the
fallback-with-warning / REQUIRE switch (:35, :54-80). What changes:

* device-resident operands run the hand-written gfx950 kernels (one launch
  per call, batched GEMM included); host operands run on the host CPU or are
  uploaded, by a host-vs-device cost model refitted for the MI355X host link;
* fp64 is native on MI355X: device-resident float64 stays on the device
  (torch / rocBLAS at fp64) instead of the reference's host bounce
  (`_fp64_host_guard`, :543-602); `gemm_fp64` (Ozaki) runs split, slice
  products and recombination all on the device;
* there is no silent fallback when the HIP library is missing on a GPU box:
  `HipLibraryError` propagates. A kernel that returns an error code
  (`HipKernelError`) falls back to torch on the same device with one
  `HipFallbackWarning` per signature, or raises under TRNBLAS_REQUIRE_HIP=1
  (TRNBLAS_REQUIRE_NKI=1 is accepted too).
"""

from __future__ import annotations

import json
import math
import os
import warnings

import torch

from .._flags import diag_flag, side_flag, trans_flag, uplo_flag
from . import _lib
from ._lib import HipKernelError, HipLibraryError  # noqa: F401  (re-exported)

_TRUE = ("1", "true", "yes", "on")


def _env_flag(*names: str) -> bool:
    return any(os.environ.get(n, "").strip().lower() in _TRUE for n in names)


_REQUIRE_HIP = _env_flag("TRNBLAS_REQUIRE_HIP", "TRNBLAS_REQUIRE_NKI")
_OFF = ("0", "false", "no", "off")


def _env_on(name: str, default: str = "1") -> bool:
    """A switch that is on unless set to 0 / false / no / off (the
    reference's convention for its default-on switches)."""
    return os.environ.get(name, default).strip().lower() not in _OFF


class HipFallbackWarning(UserWarning):
    """A HIP kernel call failed and the result was computed by torch instead
    (once per distinct error; set TRNBLAS_REQUIRE_HIP=1 to raise)."""


NkiFallbackWarning = HipFallbackWarning  # the reference's name (dispatch.py:54)

_fallback_warned: set = set()


def _warn_fallback(exc: BaseException, what: str = "HIP kernel failed — computed by torch") -> None:
    lines = str(exc).splitlines()
    key = (what, f"{type(exc).__name__}: {(lines[0] if lines else '')[:200]}")
    if key in _fallback_warned:
        return
    _fallback_warned.add(key)
    warnings.warn(
        f"{what} (set TRNBLAS_REQUIRE_HIP=1 to re-raise). First error: {key[1]}",
        HipFallbackWarning,
        stacklevel=3,
    )


def _kernel_failed(exc: Exception, what: str = "HIP kernel failed — computed by torch") -> None:
    """Re-raise `exc` unless it is a kernel error that may fall back."""
    if _REQUIRE_HIP or not isinstance(exc, HipKernelError):
        raise exc
    _warn_fallback(exc, what)


# ── backend ──────────────────────────────────────────────────────────────────

_BACKENDS = ("auto", "pytorch", "hip", "nki")
_backend = "auto"


_hip_seen = False


def has_hip() -> bool:
    """A ROCm GPU is visible to torch (does not load the op library). A
    positive answer is kept: it is asked on every call of the public API."""
    global _hip_seen
    if not _hip_seen:
        _hip_seen = bool(getattr(torch.version, "hip", None)) and torch.cuda.is_available()
    return _hip_seen


def set_backend(backend: str) -> None:
    """'auto' (HIP kernels on a ROCm GPU, else torch), 'pytorch' (torch
    everywhere) or 'hip' (the kernels always; 'nki' is an alias)."""
    global _backend
    if backend not in _BACKENDS:
        raise ValueError(f"backend must be one of {_BACKENDS}; got {backend!r}")
    if backend in ("hip", "nki"):
        if not has_hip():
            raise RuntimeError("the hip backend needs a ROCm GPU")
        _lib.load()  # fail now, loudly, if the library is missing
        backend = "hip"
    _backend = backend


def get_backend() -> str:
    return _backend


def _use_hip() -> bool:
    if _backend == "hip":
        return True
    if _backend == "pytorch":
        return False
    return has_hip()


_AUTOTUNE = _env_flag("TRNBLAS_AUTOTUNE")


def set_autotune(enabled: bool) -> None:
    """Measure, per shape bucket, which device GEMM implementation is faster
    and route by the measurement (trnblas.set_autotune; the reference's sweep
    over its own tile configurations, nki/dispatch.py:1224-1241, :2255-2325).
    The candidates here are the HIP kernel and hipBLASLt (torch.matmul) for
    16-bit operands; results persist in $TRNBLAS_AUTOTUNE_CACHE."""
    global _AUTOTUNE
    _AUTOTUNE = bool(enabled)


def get_autotune() -> bool:
    return _AUTOTUNE


def _device_synchronize() -> None:
    if torch.cuda.is_available():
        torch.cuda.synchronize()


# ── dtype policy (dispatch.py:1244-1340) ─────────────────────────────────────

_GEMM_KERNEL_DTYPES = frozenset({torch.float32, torch.bfloat16, torch.float16})
_FP32_KERNEL_DTYPES = frozenset({torch.float32})
_KERNEL_DTYPES: dict[str, frozenset] = {
    **{f"gemm_{tm}_{tk}_{tn}": _GEMM_KERNEL_DTYPES for tm, tk, tn in (
        (64, 128, 128), (64, 128, 256), (64, 128, 512),
        (128, 128, 128), (128, 128, 256), (128, 128, 512),
    )},  # fmt: skip
    "gemm_ragged": _GEMM_KERNEL_DTYPES,
    "gemm_lnc": _GEMM_KERNEL_DTYPES,
    "gemm_lnc_tn": _GEMM_KERNEL_DTYPES,
    "syrk": _GEMM_KERNEL_DTYPES,
    "mp2_energy": _FP32_KERNEL_DTYPES,
    "fused_gemm_energy": _FP32_KERNEL_DTYPES,
    "batched_pair": _FP32_KERNEL_DTYPES,
    "j_batched": _FP32_KERNEL_DTYPES,
    "pair_energy_sym": _FP32_KERNEL_DTYPES,
    "ozaki_gemm": frozenset({torch.bfloat16}),
    "ozaki_emax": frozenset({torch.int32}),
    "ozaki_split": frozenset({torch.int32, torch.float32}),
    "ozaki_emax_col": frozenset({torch.int32}),
    "ozaki_split_col": frozenset({torch.int32, torch.float32}),
}


def _check_kernel_operands(op_name: str, *tensors) -> None:
    """TypeError unless every tensor operand of kernel op `op_name` has an
    allowed dtype (the boundary backstop of dispatch.py:1278-1293)."""
    allowed = _KERNEL_DTYPES.get(op_name)
    if allowed is None:
        raise TypeError(f"trnblas: kernel op {op_name!r} has no entry in _KERNEL_DTYPES")
    dts = [t.dtype for t in tensors if isinstance(t, torch.Tensor)]
    bad = sorted({str(d) for d in dts if d not in allowed})
    if bad:
        raise TypeError(
            f"trnblas: kernel op {op_name!r} takes {sorted(str(d) for d in allowed)}; "
            f"got operand dtypes {[str(d) for d in dts]} (unsupported: {bad})"
        )


def _no_kernel_for_dtype(what: str, *tensors, takes: str = "float32/bfloat16/float16") -> None:
    """Under TRNBLAS_REQUIRE_HIP, refuse a dtype the kernels do not take."""
    if _REQUIRE_HIP:
        dts = sorted({str(t.dtype) for t in tensors})
        raise NotImplementedError(
            f"trnblas {what}: the HIP kernels take {takes}, got {dts}. "
            "Unset TRNBLAS_REQUIRE_HIP to compute in torch."
        )


_fp32_cast_warned: set = set()


def _warn_fp32_cast(op: str) -> None:
    if op in _fp32_cast_warned:
        return
    _fp32_cast_warned.add(op)
    warnings.warn(
        f"trnblas {op}: the hip backend runs float64 operands on the FP32 kernel; "
        "precision is reduced to float32 (the result keeps float64 dtype). Use "
        "set_backend('auto') for float64 accuracy, or TRNBLAS_REQUIRE_HIP=1 to raise.",
        UserWarning,
        stacklevel=3,
    )


def _as_result_dtype(out, dtype: torch.dtype):
    if isinstance(out, torch.Tensor) and out.dtype != dtype and (
        dtype.is_floating_point or dtype.is_complex
    ):
        return out.to(dtype)
    return out


def _mp2_result_dtype(T_flat, eps_occ_chunk, eps_occ_full, eps_vir) -> torch.dtype:
    dt = torch.promote_types(T_flat.dtype, eps_occ_chunk.dtype)
    return torch.promote_types(dt, torch.promote_types(eps_occ_full.dtype, eps_vir.dtype))


def _pair_result_dtype(B, eps_vir) -> torch.dtype:
    return torch.promote_types(B.dtype, eps_vir.dtype)


# ── routing (dispatch.py:633-682, re-measured for MI355X) ────────────────────
#
# Routes: 'torch' (torch where the data is), 'hip' (the kernel on device
# operands), 'host' (torch on the host CPU), 'upload' (host operands copied to
# the GPU, the kernel, the result copied back), 'aten' (torch on the GPU).
#
# Host-vs-device model, as the reference's `_host_gemm_wins` (:277-285):
# for all-host operands the host wins when
#     macs < (threads / 2) ** 0.7 * (fixed + per_byte * link_bytes),
# `fixed` the upload + launch + download floor in host multiply-adds at two
# host threads and `per_byte` the host-link cost per byte on the same scale.
# Measured on the MI355X box over 16 shapes (square 64..4096, skinny and
# tall) at 1, 2 and 16 host threads against the upload route (pageable H2D
# ~29 GB/s, pinned D2H ~57 GB/s, ~0.1 ms floor, ~65 GMAC/s per host thread);
# the exponent 0.7 carries the host's falling parallel efficiency at small
# sizes. With these constants every one of the 48 measured cases takes the
# faster route. bf16 uses the fp32 fit (its host rate was not measured).
_HOST_GEMM_MODEL_THREADS = 2
_HOST_GEMM_THREAD_EXP = 0.7
_HOST_GEMM_MODEL = {"fp32": (1.2e7, 1.0), "bf16": (1.2e7, 1.0)}
_DEVICE_GEMM_DTYPES = {torch.float32: "fp32", torch.bfloat16: "bf16", torch.float16: "fp32"}
_NATIVE_GEMM_CHOICES = ("auto", "hip", "nki", "aten", "host")


def _native_gemm_policy() -> str:
    value = os.environ.get("TRNBLAS_NATIVE_GEMM", "auto").strip().lower()
    if value not in _NATIVE_GEMM_CHOICES:
        raise ValueError(f"TRNBLAS_NATIVE_GEMM must be one of {_NATIVE_GEMM_CHOICES}; got {value!r}")
    return "hip" if value == "nki" else value


def _on_gpu(*ts) -> bool:
    return all(t.device.type == "cuda" for t in ts)


def _on_host(*ts) -> bool:
    return all(t.device.type == "cpu" for t in ts)


def _mixed_dtypes(*ts) -> bool:
    return len({t.dtype for t in ts}) > 1


def _wants_grad(*ts) -> bool:
    return torch.is_grad_enabled() and any(t.requires_grad for t in ts)


def _upload_nbytes(t: torch.Tensor) -> int:
    if t.device.type != "cpu":
        return 0
    if t.dim() >= 3 and t.stride(0) == 0:
        return _upload_nbytes(t[0])
    return t.numel() * t.element_size()


def _host_gemm_wins(macs: float, nbytes: int, dtype: torch.dtype) -> bool:
    kind = _DEVICE_GEMM_DTYPES.get(dtype)
    if kind is None:
        return True
    fixed, per_byte = _HOST_GEMM_MODEL[kind]
    scale = (max(1, torch.get_num_threads()) / _HOST_GEMM_MODEL_THREADS) ** _HOST_GEMM_THREAD_EXP
    return macs < scale * (fixed + per_byte * nbytes)


# Device-resident GEMMs under `auto` (the reference's `_lnc_gemm_wins`,
# nki/dispatch.py:707-727, picks its kernel only where it measured a win;
# re-measured here against hipBLASLt through torch.matmul on the MI355X,
# warm medians, 2-D NN / NT / TN and the C2 shapes):
#  * fp32 stays on the HIP kernel: hipBLASLt is 8-12 % faster from 2048^3 up
#    (1.1-2x below 1024^3), but on same-sign operands at K = 8192 its result
#    is 6.0e-6 |A||B| off against fp64 where the kernel's is 2.9e-7: it misses
#    the 1e-6 componentwise gate the fp32 path is held to.
#  * SYRK stays on the kernel (the triangle: 1.2-1.7x faster than the full
#    product on hipBLASLt, C2a).
#  * bf16 / fp16 go to hipBLASLt when batch * M * N >= 2^22 and K >= 512,
#    except up to 2^23 outputs with K <= 2048, where the kernel is 7-34 %
#    faster (2048^2 x 512, 2048^3, 1024 x 4096 x 2048, 2048 x 4096 x 1024,
#    NN / NT / TN / TT). hipBLASLt's time against the kernel's elsewhere:
#    0.87-0.99 at 2^22-2^23 outputs with K 4096-8192 (TN 0.96-1.05),
#    0.70-0.97 at 2896^3, 0.77-0.87 at 4096^3 (TN 1.0) and 0.73-0.87 at
#    8192^3 (the kernel on 256 x 256 tiles: NN 1043, NT 1092, TN 1010, TT
#    1022 TF/s against 1369 / 1520 / 1157 / 1371), C2b batched 0.74. The kernel also keeps the short-K
#    and long-K shapes (2048^2 x 128: 0.8x, 1024^2 x 8192 and 256 x 8192^2:
#    0.65-0.75x of hipBLASLt's time). Batched products go to hipBLASLt only
#    with contiguous operands (a transposed right operand of a 16-bit bmm is
#    avoided).
_ATEN_16BIT_MIN_MN = 1 << 22
_ATEN_16BIT_MIN_K = 512
_ATEN_16BIT_MID_MN = 1 << 23
_ATEN_16BIT_SHORT_K = 2048


def _aten_gemm_wins(a_shape, b_shape, dtype: torch.dtype, contiguous: bool, op: str = "gemm") -> bool:
    """True when a device-resident GEMM of these operands runs faster on
    hipBLASLt than on the HIP kernel at the same accuracy (table above)."""
    if op == "syrk" or dtype not in (torch.bfloat16, torch.float16):
        return False
    M, K, N = a_shape[-2], a_shape[-1], b_shape[-1]
    nb = math.prod(_lib.broadcast_shapes(tuple(a_shape[:-2]), tuple(b_shape[:-2])))
    if nb > 1 and not contiguous:
        return False
    mn = nb * M * N
    if mn < _ATEN_16BIT_MIN_MN or K < _ATEN_16BIT_MIN_K:
        return False
    return not (mn <= _ATEN_16BIT_MID_MN and K <= _ATEN_16BIT_SHORT_K)


def _dma_ready_2d(X: torch.Tensor, rows_ext: int, cols_ext: int) -> bool:
    """A 2-D 16-bit operand the GEMM kernel reads by LDS DMA in place: a
    16-byte aligned base, and a row stride and contiguous extent that are
    multiples of 8 elements (a layout the launcher copies counts by its
    copy's extent). Strides only: no copy is made."""
    s0, s1 = X.stride()
    if s1 == 1 and s0 >= cols_ext:
        return X.data_ptr() % 16 == 0 and s0 % 8 == 0 and cols_ext % 8 == 0
    if s0 == 1 and s1 >= rows_ext:
        return X.data_ptr() % 16 == 0 and s1 % 8 == 0 and rows_ext % 8 == 0
    return cols_ext % 8 == 0


# 16-bit 2-D products whose operands the DMA kernel cannot read in place,
# below the hipBLASLt bucket above: the register-staged kernel, or packing
# plus the DMA kernel, against hipBLASLt (bf16, square, measured on the
# MI355X): 255^3 38 / 30 / 50 us, 511^3 29 / 32 / 23, 767^3 38 / 34 / 28,
# 1023^3 51 / 40 / 27, 1535^3 111 / 52 / 45. From 2^26 multiply-adds on they
# go to hipBLASLt.
_ATEN_16BIT_UNREADY_MIN_MACS = 1 << 26


def _unready_16bit_to_aten(a: torch.Tensor, b: torch.Tensor, op: str) -> bool:
    if op == "syrk" or a.dtype not in (torch.bfloat16, torch.float16) or a.dim() != 2 or b.dim() != 2:
        return False
    M, K = a.shape
    N = b.shape[1]
    if M * N * K < _ATEN_16BIT_UNREADY_MIN_MACS:
        return False
    return not (_dma_ready_2d(a, M, K) and _dma_ready_2d(b, K, N))


# ── autotune: measured kernel-vs-hipBLASLt choice per shape bucket ───────────
#
# The reference times each of its tile configurations on the first call of a
# shape bucket and keeps the winner in a JSON file
# (nki/dispatch.py:1224-1241, :2249-2325). Here the candidates are the HIP
# kernel and hipBLASLt for 16-bit device GEMMs (fp32 stays on the kernel for
# accuracy, SYRK on the kernel because it computes only the triangle): on the
# first call of a bucket both run on the caller's operands (one warm-up and
# three timed calls each, HIP events on the current stream, best of three)
# and the faster one serves every later call of that bucket.

_AUTOTUNE_CACHE_FILE = os.environ.get(
    "TRNBLAS_AUTOTUNE_CACHE", os.path.join("/var/tmp", "trnblas-amd-autotune", "cache.json")
)
_autotune_mem: dict[str, str] = {}
_autotune_loaded = False
_autotune_measured = 0  # buckets timed by this process (tests read it)


def _ceil_pow2(n: int) -> int:
    p = 1
    while p < n:
        p <<= 1
    return p


def _autotune_key(a_shape, b_shape, dtype: torch.dtype, ta: bool, tb: bool, contiguous: bool) -> str:
    """Shape bucket: dtype, operand layouts and the power-of-two ceilings of
    batch, M, K, N (the reference's `_autotune_bucket` on M, K, N)."""
    M, K, N = a_shape[-2], a_shape[-1], b_shape[-1]
    nb = math.prod(_lib.broadcast_shapes(tuple(a_shape[:-2]), tuple(b_shape[:-2])))
    name = str(dtype).replace("torch.", "")
    dims = ",".join(str(_ceil_pow2(max(1, x))) for x in (nb, M, K, N))
    return f"{name},{int(ta)}{int(tb)}{int(contiguous)},{dims}"


def _load_autotune_cache() -> None:
    global _autotune_mem, _autotune_loaded
    if _autotune_loaded:
        return
    _autotune_loaded = True
    try:
        with open(_AUTOTUNE_CACHE_FILE) as f:
            raw = json.load(f)
        _autotune_mem = {str(k): str(v) for k, v in raw.items() if v in ("hip", "aten")}
    except (OSError, ValueError, AttributeError):
        _autotune_mem = {}


def _save_autotune_cache() -> None:
    try:
        d = os.path.dirname(_AUTOTUNE_CACHE_FILE)
        if d:
            os.makedirs(d, exist_ok=True)
        tmp = f"{_AUTOTUNE_CACHE_FILE}.{os.getpid()}.tmp"
        with open(tmp, "w") as f:
            json.dump(_autotune_mem, f, indent=0, sort_keys=True)
        os.replace(tmp, _AUTOTUNE_CACHE_FILE)
    except OSError:
        pass  # an unwritable cache only costs a re-measurement next process


def _time_device_call(fn, reps: int = 3) -> float:
    """Best of `reps` timed calls (ms, HIP events on the current stream)
    after one warm-up call."""
    fn()
    best = float("inf")
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        e1.synchronize()
        best = min(best, e0.elapsed_time(e1))
    return best


def _autotune_gemm_route(a: torch.Tensor, b: torch.Tensor, op: str) -> str | None:
    """'hip' or 'aten' for device operands a, b by measurement (cached per
    bucket), or None where only one candidate is admissible (the static rule
    decides)."""
    global _autotune_measured
    if op == "syrk" or a.dtype not in (torch.bfloat16, torch.float16) or a.dim() != b.dim():
        return None
    contiguous = a.is_contiguous() and b.is_contiguous()
    if a.dim() > 2 and not contiguous:
        return None  # a transposed right operand of a 16-bit bmm stays off hipBLASLt
    ta = a.dim() == 2 and a.stride(-2) == 1 and a.shape[-2] > 1
    tb = b.dim() == 2 and b.stride(-2) == 1 and b.shape[-2] > 1
    key = _autotune_key(a.shape, b.shape, a.dtype, ta, tb, contiguous)
    _load_autotune_cache()
    hit = _autotune_mem.get(key)
    if hit is not None:
        return hit
    if torch.cuda.is_current_stream_capturing():
        # no timing inside a graph capture (event syncs would break it): the
        # static rule decides, and the bucket is measured on a later eager call
        return None
    from . import kernels

    try:
        if a.dim() == 2:
            t_hip = _time_device_call(lambda: kernels.gemm(a, b))
        else:
            a3, b3, _ = _flatten_batch(a, b)
            t_hip = _time_device_call(lambda: kernels.gemm(a3, b3))
    except Exception as exc:  # noqa: BLE001
        _kernel_failed(exc)  # raises under TRNBLAS_REQUIRE_HIP
        return "aten"  # not cached: the kernel is retried in the next process
    try:
        t_aten = _time_device_call(lambda: torch.matmul(a, b))
    except Exception:  # noqa: BLE001  hipBLASLt failed: keep the kernel, uncached
        return "hip"
    choice = "aten" if t_aten < t_hip else "hip"
    _autotune_mem[key] = choice
    _autotune_measured += 1
    _save_autotune_cache()
    return choice


def _gemm_route(*tensors, op: str = "gemm", macs: float | None = None, nbytes: int | None = None):
    """'torch', 'hip', 'host', 'upload' or 'aten' for a GEMM-family call."""
    if not _use_hip() or _mixed_dtypes(*tensors) or _wants_grad(*tensors):
        return "torch"
    if any(t.dtype not in _GEMM_KERNEL_DTYPES for t in tensors):
        _no_kernel_for_dtype(op, *tensors)
        return "torch"  # float64 / complex / integer: torch where the data is
    policy = _native_gemm_policy()
    if _on_gpu(*tensors):
        if policy == "aten":
            return "aten"
        if policy == "auto" and _backend == "auto" and len(tensors) >= 2:
            a, b = tensors[0], tensors[1]
            tuned = _autotune_gemm_route(a, b, op) if _AUTOTUNE else None
            if tuned is not None:
                return tuned
            if _aten_gemm_wins(a.shape, b.shape, a.dtype, a.is_contiguous() and b.is_contiguous(), op):
                return "aten"
            if _unready_16bit_to_aten(a, b, op):
                return "aten"
        return "hip"
    if not _on_host(*tensors):
        return "upload"  # mixed residency: compute on the GPU operand's device
    if policy == "host":
        return "host"
    if _backend == "hip" or policy in ("hip", "aten"):
        return "upload"
    if macs is None:
        a, b = tensors[0], tensors[1]
        macs = a.shape[-2] * a.shape[-1] * b.shape[-1] * max(1, math.prod(a.shape[:-2]))
        nbytes = (
            sum(_upload_nbytes(t) for t in tensors[:2])
            + (macs // max(1, a.shape[-1])) * a.element_size()
        )
    return "host" if _host_gemm_wins(macs, nbytes, tensors[0].dtype) else "upload"


def _gpu_device(*ts) -> torch.device:
    for t in ts:
        if isinstance(t, torch.Tensor) and t.device.type == "cuda":
            return t.device
    return torch.device("cuda", torch.cuda.current_device())


def _to(t, dev):
    return t if t is None or t.device == dev else t.to(dev, non_blocking=False)


_PINNED_OUTPUT_MIN_BYTES = 1 << 20


def _pinned_output_enabled() -> bool:
    """TRNBLAS_PINNED_OUTPUT=0 (or false / no / off) turns pinned results off
    (nki/dispatch.py:2052-2060); read at every call, as the reference does."""
    return _env_on("TRNBLAS_PINNED_OUTPUT")


def _to_host(t: torch.Tensor, orig: torch.device) -> torch.Tensor:
    """A device result back on the host device `orig`: results of 1 MiB and
    more into fresh pinned memory (device-to-host copies from pageable memory
    run ~4 GB/s on the MI355X host, from pinned ~10x faster; the reference's
    `_host_empty` / `_to_host`, nki/dispatch.py:2055-2101, makes the same
    choice), unless TRNBLAS_PINNED_OUTPUT turns that off."""
    if orig.type != "cpu" or t.device.type == "cpu":
        return t.to(orig)
    if t.numel() * t.element_size() < _PINNED_OUTPUT_MIN_BYTES or not _pinned_output_enabled():
        return t.cpu()
    out = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
    out.copy_(t)
    return out


# ── GEMM family ──────────────────────────────────────────────────────────────


def _fused_epilogue_ok(C, beta, shape, dtype, device) -> bool:
    """True when beta * C can be fused into the kernel's store: C absent /
    beta 0, or C of the result dtype and device broadcasting to `shape`."""
    if C is None or beta == 0.0:
        return True
    if C.dtype == dtype and C.device == device and tuple(C.shape) == tuple(shape):
        return True
    return (
        C.dtype == dtype
        and C.device == device
        and _lib.broadcast_shapes(tuple(shape), tuple(C.shape)) == tuple(shape)
    )


def _torch_scale_add(result, alpha, beta, C):
    """alpha * result + beta * C out of place (level3.py:42-66 semantics)."""
    result = alpha * result if alpha != 1.0 else result
    return result + beta * C if (C is not None and beta != 0.0) else result


def hip_gemm(A, B, alpha=1.0, beta=0.0, C=None) -> torch.Tensor:
    """alpha * A @ B + beta * C on the GPU kernel; A, B 2-D or 3-D device
    tensors (torch.matmul broadcasting of one batch dim)."""
    from . import kernels

    if A.dim() == 3 and B.dim() == 2:
        B = B.unsqueeze(0)
    elif A.dim() == 2 and B.dim() == 3:
        A = A.unsqueeze(0)
    out_shape = (
        (A.shape[0] if A.dim() == 3 else None),
        A.shape[-2],
        B.shape[-1],
    )
    if A.dim() == 3:
        out_shape = (max(A.shape[0], B.shape[0]), A.shape[-2], B.shape[-1])
    else:
        out_shape = (A.shape[0], B.shape[1])
    if _fused_epilogue_ok(C, beta, out_shape, A.dtype, A.device):
        return kernels.gemm(A, B, alpha, beta, C)
    return _torch_scale_add(kernels.gemm(A, B, 1.0, 0.0, None), alpha, beta, C)


def _flatten_batch(A, B):
    """A (..., M, K), B (..., K, N) -> 3-D operands with one broadcast batch
    dim (views when possible), and the broadcast batch shape."""
    batch = _lib.broadcast_shapes(A.shape[:-2], B.shape[:-2])
    nb = math.prod(batch)

    def as3(X):
        if X.dim() == 2:
            return X.unsqueeze(0)
        if tuple(X.shape[:-2]) == tuple(batch):
            return X.reshape(nb, *X.shape[-2:])
        if math.prod(X.shape[:-2]) == 1:
            return X.reshape(1, *X.shape[-2:])
        return X.expand(*batch, *X.shape[-2:]).reshape(nb, *X.shape[-2:])

    return as3(A), as3(B), batch


def nki_gemm(A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    """A @ B for 2-D operands (dispatch.py:1526-1551): the HIP kernel for
    device operands, torch otherwise (see `_gemm_route`)."""
    route = _gemm_route(A, B)
    if route == "hip":
        try:
            return hip_gemm(A, B)
        except Exception as exc:  # noqa: BLE001
            _kernel_failed(exc)
            return torch.matmul(A, B)
    if route == "upload":
        dev = _gpu_device(A, B)
        orig = A.device
        try:
            return _to_host(hip_gemm(_to(A, dev), _to(B, dev)), orig)
        except Exception as exc:  # noqa: BLE001
            _kernel_failed(exc)
            return torch.matmul(A, B)
    return torch.matmul(A, B)


def nki_batched_gemm(A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    """torch.matmul batch semantics (dispatch.py:1384-1427) in one launch."""
    if A.dim() < 2 or B.dim() < 2:
        return torch.matmul(A, B)
    batch = _lib.broadcast_shapes(A.shape[:-2], B.shape[:-2])
    if math.prod(batch) == 0:
        return torch.matmul(A, B)
    route = _gemm_route(A, B, op="batched_gemm")
    if route not in ("hip", "upload"):
        return torch.matmul(A, B)
    dev = _gpu_device(A, B)
    orig = A.device
    try:
        a3, b3, batch = _flatten_batch(_to(A, dev), _to(B, dev))
        out = hip_gemm(a3, b3).reshape(*batch, A.shape[-2], B.shape[-1])
        return _to_host(out, orig) if orig != dev else out
    except Exception as exc:  # noqa: BLE001
        _kernel_failed(exc)
        return torch.matmul(A, B)


_F32 = torch.float32
_gemm_fn = None  # the library's trnblas_hip_gemm, once loaded
_kernels = None  # the kernels module, once imported


def gemm_fast(alpha, A, B, beta, C, transA, transB):
    """level3.gemm's common case without the general routing: 2-D fp32
    operands on one GPU, no gradient, the native GEMM policy auto or hip,
    each operand row-major or a transposed row-major view that the kernel
    reads in place (16-byte aligned, leading dimension and contiguous extent
    multiples of 4), C absent or of the result's shape with unit column
    stride. Returns alpha op(A) op(B) + beta C, or None (the general path
    then decides, as for every other call; also on a library error, which
    the general path reports). The route is the one `_gemm_route` gives
    these operands ("hip"); the host time per call is about half of the
    general path's."""
    global _gemm_fn, _kernels
    kern = _kernels
    if kern is None:
        from . import kernels as kern

        _kernels = kern
    if (
        type(transA) is not bool
        or type(transB) is not bool
        or A.dtype is not _F32
        or B.dtype is not _F32
        or not A.is_cuda
        or A.dim() != 2
        or B.dim() != 2
        or _backend == "pytorch"
        or kern._launch_probe is not None
    ):
        return None
    dev = A.get_device()
    if B.get_device() != dev or (torch.is_grad_enabled() and (A.requires_grad or B.requires_grad)):
        return None
    policy = os.environ.get("TRNBLAS_NATIVE_GEMM")
    if policy is not None and policy.strip().lower() not in ("auto", "hip", "nki"):
        return None
    if _backend == "auto" and not has_hip():
        return None
    # op(A) (M, K) and op(B) (K, N) from the stored strides: trans flag of
    # the C ABI (the operand is stored transposed) and leading dimension
    ar, ac = A.shape
    br, bc = B.shape
    M, K = (ac, ar) if transA else (ar, ac)
    K2, N = (bc, br) if transB else (br, bc)
    if K != K2 or M == 0 or N == 0 or K == 0:
        return None
    a0, a1 = A.stride()
    b0, b1 = B.stride()
    if a1 == 1 and a0 >= ac:  # stored row-major (ar, ac)
        ta, lda, aext = transA, a0, ac
    elif a0 == 1 and a1 >= ar:  # stored column-major: a transposed view
        ta, lda, aext = not transA, a1, ar
    else:
        return None
    if b1 == 1 and b0 >= bc:
        tb, ldb, bext = transB, b0, bc
    elif b0 == 1 and b1 >= br:
        tb, ldb, bext = not transB, b1, br
    else:
        return None
    pa, pb = A.data_ptr(), B.data_ptr()
    if (pa | pb) & 15 or (lda | ldb | aext | bext) & 3:
        return None
    c, ldc, cb = 0, N, 0.0
    if C is not None and beta != 0.0:
        if (
            C.dtype is not _F32
            or not C.is_cuda
            or C.get_device() != dev
            or C.dim() != 2
            or C.shape[0] != M
            or C.shape[1] != N
            or C.stride(1) != 1
            or C.stride(0) < N
            or (torch.is_grad_enabled() and C.requires_grad)
        ):
            return None
        c, ldc, cb = C.data_ptr(), C.stride(0), float(beta)
    fn = _gemm_fn
    if fn is None:
        fn = _gemm_fn = _lib.load().trnblas_hip_gemm
    ws = kern.gemm_workspace(A.device)
    D = torch.empty((M, N), dtype=_F32, device=A.device)
    rc = fn(0, int(ta), int(tb), M, N, K, float(alpha), pa, lda, 0, pb, ldb, 0, cb, c or None, ldc, 0,
            D.data_ptr(), N, 0, 1, ws.data_ptr(), ws.numel(), torch._C._cuda_getCurrentRawStream(dev))  # fmt: skip
    return D if rc >= 0 else None


def gemm_scaled(alpha, a, b, beta, C):
    """alpha * a @ b + beta * C with the epilogue fused into the kernel when
    the route is a kernel route (level3.gemm / batched_gemm)."""
    if a.dim() < 2 or b.dim() < 2:
        return _torch_scale_add(torch.matmul(a, b), alpha, beta, C)
    flat = a.dim() == 2 and b.dim() == 2
    batch = () if flat else _lib.broadcast_shapes(a.shape[:-2], b.shape[:-2])
    route = _gemm_route(a, b, op="gemm" if flat else "batched_gemm")
    if route not in ("hip", "upload") or math.prod(batch) == 0 or len(batch) > 1:
        if route in ("hip", "upload") and len(batch) > 1:
            return _torch_scale_add(nki_batched_gemm(a, b), alpha, beta, C)
        return _torch_scale_add(torch.matmul(a, b), alpha, beta, C)
    dev = _gpu_device(a, b, *(() if C is None else (C,)))
    orig = a.device
    try:
        ad, bd = _to(a, dev), _to(b, dev)
        Cd = None if (C is None or beta == 0.0) else (C.to(dev) if C.device != dev else C)
        out = hip_gemm(ad, bd, alpha, beta, Cd)
        return _to_host(out, orig) if orig != dev else out
    except Exception as exc:  # noqa: BLE001
        _kernel_failed(exc)
        return _torch_scale_add(torch.matmul(a, b), alpha, beta, C)


# ── SYRK ─────────────────────────────────────────────────────────────────────


def _symmetrize(r: torch.Tensor) -> torch.Tensor:
    """0.5 * (r + r^T) (dispatch.py:3178-3199 values)."""
    return 0.5 * (r + r.mT)


def _solve_dtype(*ts: torch.Tensor) -> torch.dtype:
    """The arithmetic of a triangular solve / Cholesky: half types in fp32."""
    dt = torch.promote_types(ts[0].dtype, ts[-1].dtype)
    return torch.float32 if dt in (torch.bfloat16, torch.float16) else dt


def nki_trsm(
    A: torch.Tensor,
    B: torch.Tensor,
    side: str = "left",
    uplo: str = "upper",
    trans: bool = False,
    diag: str = "nonunit",
    alpha: float = 1.0,
) -> torch.Tensor:
    """Triangular solve with multiple right-hand sides: op(A) X = alpha B
    (side "left") or X op(A) = alpha B (side "right"), op(A) = A or A^T.
    Only the `uplo` triangle of A is read; diag "unit" takes its diagonal as
    ones (the reference body, nki/dispatch.py:1707-1738). The reference's
    device route is a blocked solve, diagonal panels by
    torch.linalg.solve_triangular and updates by its GEMM kernel
    (`_nki_trsm_left`, :1740-1799; Trainium has no fp64). On MI355X a
    device-resident 2-D solve runs the HIP blocked solve (`_trsm_hip`:
    every 128 x 128 diagonal block inverted at once by
    trnblas_hip_tri_inv_blocks, then block solves and updates as GEMMs on
    the fp64 or fp32 MFMA kernels) in the operands' own precision, float64
    included; bf16 / fp16 solve in fp32 and return in B's dtype, as the
    reference's host route does. Host operands, complex or batched
    right-hand sides, and calls that need gradients take torch's
    `solve_triangular` (differentiable in A and B)."""
    side, uplo, diag = side_flag(side), uplo_flag(uplo), diag_flag(diag)
    trans = trans_flag(trans)
    if A.dim() != 2 or A.shape[0] != A.shape[1]:
        raise ValueError(f"trsm: A must be square; got {tuple(A.shape)}")
    n = A.shape[0]
    need = B.shape[-2] if side == "left" else B.shape[-1]
    if B.dim() < 2 or need != n:
        raise ValueError(f"trsm: A {tuple(A.shape)} does not match B {tuple(B.shape)} for side={side!r}")
    if not (A.is_floating_point() or A.is_complex()) or not (B.is_floating_point() or B.is_complex()):
        raise NotImplementedError(f"trsm: expected floating point operands; got {A.dtype}, {B.dtype}")
    cdt = _solve_dtype(A, B)
    if (
        _use_hip()
        and A.is_cuda
        and B.is_cuda
        and A.device == B.device
        and B.dim() == 2
        and cdt in (torch.float32, torch.float64)
        and not _wants_grad(A, B)
    ):
        try:
            return _trsm_hip(A.to(cdt), B.to(cdt), side, uplo, trans, diag, alpha).to(B.dtype)
        except Exception as exc:  # noqa: BLE001
            _kernel_failed(exc)
    mat = A.mT if trans else A  # the uplo triangle of A is the other one of A^T
    upper = (uplo == "upper") != trans
    rhs = B.to(cdt) if alpha == 1.0 else alpha * B.to(cdt)
    X = torch.linalg.solve_triangular(
        mat.to(cdt), rhs, upper=upper, left=side == "left", unitriangular=diag == "unit"
    )
    return X.to(B.dtype)


def _trsm_hip(A, B, side, uplo, trans, diag, alpha):
    """op(A) X = alpha B (left) or X op(A) = alpha B (right) on the device,
    float32 / float64, through the native blocked solve (trnblas_hip_trsm:
    the reference's `_nki_trsm_left`, nki/dispatch.py:1740-1799, with its
    per-block solve_triangular replaced by one launch that inverts every
    diagonal block). A right solve is the left solve op(A)^T X^T = alpha B^T:
    the transposed views go to the driver as they are."""
    from . import kernels

    if side == "left":
        M, rhs = (A.mT if trans else A), B
        upper = (uplo == "upper") != trans
    else:
        M, rhs = (A if trans else A.mT), B.mT
        upper = (uplo == "upper") == trans
    out = torch.empty(B.shape, dtype=B.dtype, device=B.device)
    kernels.trsm(M, rhs, upper, diag == "unit", alpha, out if side == "left" else out.mT)
    return out


def _metric_inv_half_blocked(J: torch.Tensor) -> torch.Tensor:
    """X = L^-T of a real SPD J on the ROCm device, in fp64, by the native
    driver trnblas_hip_metric_inv_half: a right-looking blocked Cholesky
    (128-wide diagonal blocks factored and inverted by one kernel each,
    fp64 MFMA GEMM panels and lower-triangle trailing updates, the trailing
    update on a second stream beside the next diagonal block), then L^-1 by
    recursive doubling over block halves, one batched GEMM pair per level,
    and its transpose. Returns float64."""
    from . import kernels

    X, info = kernels.metric_inv_half(J.to(torch.float64))
    bad = int(info)  # one small device-to-host read
    if bad != 0:
        raise torch.linalg.LinAlgError(
            f"metric Cholesky failed: leading minor of order {bad} is not positive-definite"
        )
    return X


_METRIC_SOLVE_CHOICES = ("auto", "host", "device")


def _metric_solve_route(J: torch.Tensor) -> str:
    """'host' or 'device' for `nki_metric_inv_half` (the reference's
    `_metric_solve_route`, nki/dispatch.py:1833-1849, and its
    TRNBLAS_METRIC_SOLVE=auto|host|device override). "auto" keeps a device J
    on the device at every size: on the MI355X the fp64 HIP driver beats the
    host's LAPACK from the smallest metrics up (naux 4096: 2.8 ms against
    139-217 ms), where the reference's Trainium route sends naux <= 1024 to
    the host. "host" computes the factor with host LAPACK in fp64 and copies
    it back. A host J takes host LAPACK whatever the setting."""
    choice = os.environ.get("TRNBLAS_METRIC_SOLVE", "auto").strip().lower()
    if choice not in _METRIC_SOLVE_CHOICES:
        raise ValueError(
            f"TRNBLAS_METRIC_SOLVE must be one of {_METRIC_SOLVE_CHOICES}; got {choice!r}"
        )
    if not J.is_cuda:
        return "device"  # plain torch on the host (host LAPACK), as the reference
    return "host" if choice == "host" else "device"


def nki_metric_inv_half(J: torch.Tensor) -> torch.Tensor:
    """Cholesky inverse factor X = L^-T of an SPD metric J = L L^T, so
    X X^T = J^-1 and `A @ X` is the density-fitting metric contraction
    (nki/dispatch.py:1854-1905). On MI355X a real J on the device is factored
    and inverted there in fp64 (`_metric_inv_half_blocked`: the native HIP
    driver, diagonal-block kernels and fp64 MFMA GEMMs), where the reference sends device
    metrics to host LAPACK or runs torch.linalg.cholesky + trsm in the
    metric's precision; complex metrics and host tensors take torch's
    Cholesky and triangular solve (host LAPACK for host tensors, the
    reference's own host route). The result has J's dtype and device; X is
    exactly upper triangular."""
    if not (J.is_floating_point() or J.is_complex()):
        # every route of the reference raises for integer metrics (#86)
        raise NotImplementedError(
            f"metric_inv_half: expected a floating point or complex tensor; got {J.dtype}"
        )
    if J.dim() != 2 or J.shape[0] != J.shape[1]:
        raise ValueError(f"metric_inv_half: J must be square; got {tuple(J.shape)}")
    route = _metric_solve_route(J)
    if route == "host":
        # the reference's host route (nki/dispatch.py:1854-1870): fp64 LAPACK
        # on the host, the factor copied back in J's dtype
        Jd = J.detach().to("cpu", torch.float64)
        L, info = torch.linalg.cholesky_ex(Jd)
        if int(info) != 0:
            raise torch.linalg.LinAlgError(
                f"metric Cholesky failed: leading minor of order {int(info)} is not positive-definite"
            )
        eye = torch.eye(Jd.shape[0], dtype=torch.float64)
        X = torch.linalg.solve_triangular(L.mT, eye, upper=True).contiguous()
        return X.to(dtype=J.dtype).to(J.device)
    if route == "device" and J.is_cuda and J.is_floating_point():
        return _metric_inv_half_blocked(J).to(J.dtype)
    cdt = _solve_dtype(J)
    L, info = torch.linalg.cholesky_ex(J.to(cdt))
    if int(info) != 0:  # one small device-to-host read
        raise torch.linalg.LinAlgError(
            f"metric Cholesky failed: leading minor of order {int(info)} is not positive-definite"
        )
    eye = torch.eye(J.shape[0], dtype=cdt, device=J.device)
    # L^-T: solve L^T X = I (the reference's trsm(L, I, uplo="lower", trans=True))
    X = torch.linalg.solve_triangular(L.mT, eye, upper=True)
    return X.to(J.dtype)


def nki_syrk(A: torch.Tensor, symmetrize: bool = False) -> torch.Tensor:
    """A @ A^T (dispatch.py:1554-1594); the kernel computes the lower
    triangle only and mirrors it, so the result is exactly symmetric."""
    M, K = A.shape
    route = _gemm_route(A, op="syrk", macs=M * M * K, nbytes=(M * K + M * M) * A.element_size())
    if route in ("hip", "upload"):
        from . import kernels

        dev = _gpu_device(A)
        try:
            return _to_host(kernels.syrk(_to(A, dev)), A.device)
        except Exception as exc:  # noqa: BLE001
            _kernel_failed(exc)
    r = torch.matmul(A, A.mT)
    return _symmetrize(r) if symmetrize else r


def hip_syrk(alpha, A, beta, C, trans: bool, uplo: str) -> torch.Tensor | None:
    """The fused SYRK for device (or uploaded) operands, or None when the
    route is not a kernel route. C is n x n (only its `uplo` triangle read)."""
    n = A.shape[1] if trans else A.shape[0]
    k = A.shape[0] if trans else A.shape[1]
    ts = (A,) if C is None or beta == 0.0 else (A, C)
    route = _gemm_route(*ts, op="syrk", macs=n * n * k, nbytes=(n * k + 2 * n * n) * A.element_size())
    if route not in ("hip", "upload"):
        return None
    from . import kernels

    dev = _gpu_device(*ts)
    orig = A.device
    try:
        Cd = None if C is None or beta == 0.0 else _to(C, dev)
        out = kernels.syrk(_to(A, dev), alpha, beta if Cd is not None else 0.0, Cd, trans, uplo)
        return _to_host(out, orig) if orig != dev else out
    except Exception as exc:  # noqa: BLE001
        _kernel_failed(exc)
        return None


def hip_syrk_checked(alpha, A, beta, C, trans: bool, uplo: str):
    """SYRK with beta != 0 and an n x n C of A's dtype whose referenced
    triangle is decided on the device (`kernels.syrk_checked`): (D, the uplo
    triangle has an off-diagonal nonzero, the other triangle has one), or
    None when the route is not a kernel route."""
    n = A.shape[1] if trans else A.shape[0]
    k = A.shape[0] if trans else A.shape[1]
    route = _gemm_route(A, C, op="syrk", macs=n * n * k, nbytes=(n * k + 2 * n * n) * A.element_size())
    if route not in ("hip", "upload"):
        return None
    from . import kernels

    dev = _gpu_device(A, C)
    orig = A.device
    try:
        out, mine, theirs = kernels.syrk_checked(_to(A, dev), alpha, beta, _to(C, dev), trans, uplo)
        return (_to_host(out, orig) if orig != dev else out), mine, theirs
    except Exception as exc:  # noqa: BLE001
        _kernel_failed(exc)
        return None


# ── DF-MP2 energies ──────────────────────────────────────────────────────────

_PAIR_ENERGY_CHOICES = ("auto", "hip", "sym", "aten", "legacy")


def _pair_energy_choice() -> str:
    c = os.environ.get("TRNBLAS_PAIR_ENERGY", "auto").strip().lower()
    if c not in _PAIR_ENERGY_CHOICES:
        raise ValueError(f"TRNBLAS_PAIR_ENERGY must be one of {_PAIR_ENERGY_CHOICES}; got {c!r}")
    return c


def _energy_operands(what: str, data: tuple, eps: tuple):
    """fp32 operands for an energy kernel, or None to run torch
    (dispatch.py:1296-1325): bf16 / fp16 upcast exactly; float64 under
    `auto` runs torch at fp64, under `hip` is cast with a warning."""
    ts = (*data, *eps)
    bad = [t for t in ts if t.dtype not in _GEMM_KERNEL_DTYPES]
    if bad:
        _no_kernel_for_dtype(what, *ts, takes="float32 amplitudes and orbital energies")
        if not (_backend == "hip" and all(t.dtype == torch.float64 for t in bad)):
            return None
        _warn_fp32_cast(what)
    f32 = torch.float32
    return tuple(t.to(f32) for t in data), tuple(t.to(f32) for t in eps)


def _torch_batched_pair_energy(B, eps_occ, eps_vir) -> torch.Tensor:
    """The pytorch backend of the batched pair energy (dispatch.py:2514-2533)."""
    e = torch.zeros((), dtype=B.dtype, device=B.device)
    for i in range(B.shape[0]):
        for j in range(B.shape[0]):
            T = B[i] @ B[j].T
            D = float(eps_occ[i]) + float(eps_occ[j]) - eps_vir.unsqueeze(1) - eps_vir.unsqueeze(0)
            e = e + (T * (2.0 * T - T.T) / D).sum()
    return e


def _torch_chunked_pair_energy(B, eps_occ, eps_vir, mem_budget_bytes: int = 1_500_000_000):
    """Chunked GEMM + torch reduction (dispatch.py:2706-2728): the `aten`
    route, and the unfused GPU baseline of the fused kernel."""
    nocc, nvir, naux = B.shape
    i_block = max(1, min(nocc, int(mem_budget_bytes // (4 * nvir * nocc * nvir))))
    flat = B.reshape(nocc * nvir, naux)
    eo2 = eps_occ.view(nocc, 1, 1, 1) + eps_occ.view(1, nocc, 1, 1)
    ev2 = eps_vir.view(1, 1, nvir, 1) + eps_vir.view(1, 1, 1, nvir)
    e = torch.zeros((), dtype=B.dtype, device=B.device)
    for i0 in range(0, nocc, i_block):
        i1 = min(i0 + i_block, nocc)
        T = (flat[i0 * nvir : i1 * nvir] @ flat.T).reshape(i1 - i0, nvir, nocc, nvir)
        T = T.permute(0, 2, 1, 3)
        e = e + (T * (2.0 * T - T.transpose(-2, -1)) / (eo2[i0:i1] - ev2)).sum()
    return e


# Fused kernel vs the unfused chunked path (hipBLASLt GEMM + torch
# elementwise) under `auto`, as the reference's row-flop / SBUF rule
# (nki/dispatch.py:2680-2703) re-measured for MI355X: over 90 small shapes
# (nocc 2, 4, 8, 16, 32, 64 x nvir 32, 96, 192, 320, 448 x naux 128, 512,
# 1536) the fused fp16x3 kernel loses in 10, all at naux 1536 where its work
# items (squares of pairs of occupied rows x 96-row tile pairs) fill a
# fraction of the 256 CUs, so one item's k-steps (~1.9 us each when few
# items share the chip, two passes off the tile diagonal) form the whole
# critical path; the unfused path costs a ~0.115 ms floor plus its
# ordered-pair GEMM (~100 TFLOP/s) and six fp32 passes over T (~3 TB/s).
# The model below picks the faster route in 87 of the 90 cases (mean loss
# 0.16 %). At C3 / C4 it keeps the fused kernel by a wide margin.
_PE_STEP_MS = 1.9e-3
_PE_FUSED_FLOOR_MS = 0.05
_PE_UNFUSED_FLOOR_MS = 0.115
_PE_UNFUSED_GEMM_FLOPS = 100e12
_PE_UNFUSED_T_BYTES_PER_S = 3e12
_PE_TILE = 96
_PE_CUS = 256


def _pair_energy_estimates(nocc: int, nvir: int, naux: int) -> tuple[float, float]:
    """(fused, unfused) estimated milliseconds for B (nocc, nvir, naux)."""
    nb = -(-nvir // _PE_TILE)
    nq = nb * (nb + 1) // 2
    nb2 = (nocc + 1) // 2
    squares = nb2 * (nb2 + 1) // 2  # pairs i <= j, up to four per item
    nk = -(-naux // 32)
    steps = (nk * nb + 2 * nk * (nq - nb)) / nq  # mean k-steps per item
    fused = _PE_FUSED_FLOOR_MS + math.ceil(squares * nq / _PE_CUS) * steps * _PE_STEP_MS
    m = nocc * nvir
    unfused = (
        _PE_UNFUSED_FLOOR_MS
        + 2.0 * m * m * naux / _PE_UNFUSED_GEMM_FLOPS * 1e3
        + 24.0 * m * m / _PE_UNFUSED_T_BYTES_PER_S * 1e3
    )
    return fused, unfused


def _pair_energy_route(B) -> str:
    """'hip' (fused kernel), 'aten' (chunked torch on the GPU) or 'torch'."""
    choice = _pair_energy_choice()
    if not _use_hip():
        return "torch"
    if choice == "aten":
        return "aten" if B.device.type == "cuda" else "torch"
    if choice == "auto" and _backend == "auto" and B.device.type == "cuda" and B.dim() == 3:
        fused, unfused = _pair_energy_estimates(*B.shape)
        if unfused < fused:
            return "aten"
    return "hip"


def nki_batched_pair_energy(B: torch.Tensor, eps_occ: torch.Tensor, eps_vir: torch.Tensor):
    """Total DF-MP2 pair energy over all nocc^2 ordered pairs
    (dispatch.py:2536-2569): one fused HIP launch for the i <= j walk.
    B (nocc, nvir, naux), eps_occ (nocc,), eps_vir (nvir,). Returns a 0-d
    tensor of the pytorch backend's dtype on B's device."""
    dt = _pair_result_dtype(B, eps_vir)
    route = _pair_energy_route(B)
    if route == "torch":
        return _torch_batched_pair_energy(B, eps_occ, eps_vir)
    if route == "aten":
        return _torch_chunked_pair_energy(B, eps_occ, eps_vir)
    feeds = _energy_operands("batched_pair_energy", (B,), (eps_occ, eps_vir))
    if feeds is None:
        if B.device.type == "cuda":
            return _torch_chunked_pair_energy(B, eps_occ, eps_vir)
        return _torch_batched_pair_energy(B, eps_occ, eps_vir)
    (Bk,), (eo, ev) = feeds
    from . import kernels

    dev = _gpu_device(B, eps_occ, eps_vir)
    try:
        e = kernels.pair_energy_sym(Bk.to(dev), eo.to(dev), ev.to(dev))
        return _as_result_dtype(e, dt).to(B.device)
    except Exception as exc:  # noqa: BLE001
        _kernel_failed(exc, "pair energy kernel failed — computed by torch")
        return _torch_chunked_pair_energy(B, eps_occ, eps_vir)


def nki_fused_gemm_energy(b_i, b_j, eps_occ_i: float, eps_occ_j: float, eps_vir):
    """One pair's energy (dispatch.py:3049-3164)."""
    dt = torch.promote_types(_pair_result_dtype(b_i, eps_vir), b_j.dtype)

    def torch_ref():
        T = b_i @ b_j.T
        D = eps_occ_i + eps_occ_j - eps_vir.unsqueeze(1) - eps_vir.unsqueeze(0)
        return (T * (2.0 * T - T.T) / D).sum()

    if not _use_hip():
        return torch_ref()
    feeds = _energy_operands("fused_gemm_energy", (b_i, b_j), (eps_vir,))
    if feeds is None:
        return torch_ref()
    (bi, bj), (ev,) = feeds
    from . import kernels

    dev = _gpu_device(b_i, b_j, eps_vir)
    try:
        eo = torch.tensor([float(eps_occ_i), float(eps_occ_j)], dtype=torch.float32, device=dev)
        zero = torch.zeros(1, dtype=torch.int32)
        e = kernels.pair_energies(
            bi.to(dev).unsqueeze(0), bj.to(dev).unsqueeze(0), eo[:1], eo[1:], ev.to(dev), zero, zero
        )[0]
        return _as_result_dtype(e, dt).to(b_i.device)
    except Exception as exc:  # noqa: BLE001
        _kernel_failed(exc)
        return torch_ref()


def _torch_mp2_energy(T_flat, eps_occ_chunk, eps_occ_full, eps_vir):
    """dispatch.py:1440-1453: T (ic, nocc, nvir, nvir) from T_flat, reduced."""
    ic, nocc, nvir = eps_occ_chunk.shape[0], eps_occ_full.shape[0], eps_vir.shape[0]
    T = T_flat.reshape(ic, nvir, nocc, nvir).permute(0, 2, 1, 3)
    D = (
        eps_occ_chunk.view(ic, 1, 1, 1)
        + eps_occ_full.view(1, nocc, 1, 1)
        - eps_vir.view(1, 1, nvir, 1)
        - eps_vir.view(1, 1, 1, nvir)
    )
    return (T * (2.0 * T - T.transpose(-2, -1)) / D).sum()


def nki_mp2_energy(T_flat, eps_occ_chunk, eps_occ_full, eps_vir):
    """The energy of a precomputed amplitude block (dispatch.py:1456-1489):
    one HBM-bound HIP reduction."""
    if not _use_hip():
        return _torch_mp2_energy(T_flat, eps_occ_chunk, eps_occ_full, eps_vir)
    feeds = _energy_operands("mp2_energy", (T_flat,), (eps_occ_chunk, eps_occ_full, eps_vir))
    if feeds is None:
        return _torch_mp2_energy(T_flat, eps_occ_chunk, eps_occ_full, eps_vir)
    (t,), (eoc, eof, ev) = feeds
    dt = _mp2_result_dtype(T_flat, eps_occ_chunk, eps_occ_full, eps_vir)
    from . import kernels

    dev = _gpu_device(T_flat, eps_occ_chunk, eps_occ_full, eps_vir)
    try:
        e = kernels.mp2_energy_pairs(t.to(dev), eoc.to(dev), eof.to(dev), ev.to(dev)).sum()
        return _as_result_dtype(e, dt).to(T_flat.device)
    except Exception as exc:  # noqa: BLE001
        _kernel_failed(exc)
        return _torch_mp2_energy(T_flat, eps_occ_chunk, eps_occ_full, eps_vir)


# ── Ozaki fp64-class GEMM ────────────────────────────────────────────────────


def _ozaki_route() -> str:
    """'kernel' or 'torch' (fp64 matmul where the data is) for gemm_fp64
    (dispatch.py:761-774)."""
    return "kernel" if _use_hip() else "torch"


_oz_split_noted = False


def _note_ozaki_device_split() -> None:
    """TRNBLAS_OZAKI_DEVICE_SPLIT=0 keeps the reference's split on the host
    (nki/dispatch.py:853-862), a Trainium workaround for its missing fp64.
    Here the split is native fp64 on the device with the same digits, so
    the switch has no effect; say so once instead of ignoring it silently."""
    global _oz_split_noted
    if not _oz_split_noted and not _env_on("TRNBLAS_OZAKI_DEVICE_SPLIT"):
        _oz_split_noted = True
        warnings.warn(
            "TRNBLAS_OZAKI_DEVICE_SPLIT=0 has no effect on ROCm: gemm_fp64 always splits on "
            "the device in native fp64, into the same digits as the host split",
            UserWarning,
            stacklevel=3,
        )


def nki_gemm_fp64(a: torch.Tensor, b: torch.Tensor, slices: int, mode: str | None = None) -> torch.Tensor:
    """fp64 a @ b by the Ozaki split on the device (dispatch.py:958-980).
    a (M, K), b (K, N) real tensors (any float dtype; computed as fp64).
    mode: "fast", "exact" or None (ozaki.default_mode()). Non-finite operands
    take a plain fp64 matmul on the device."""
    from .. import ozaki

    k = ozaki.check_slices(slices)
    mode = ozaki.check_mode(mode)
    _note_ozaki_device_split()
    if _ozaki_route() == "torch":
        return torch.matmul(a.double(), b.double())
    dev = _gpu_device(a, b)
    ad = a.to(dev, torch.float64)
    bd = b.to(dev, torch.float64)
    try:
        return ozaki.run_device(ad, bd, k, mode)
    except ozaki.OzakiNonFinite:
        return torch.matmul(ad, bd)
    except Exception as exc:  # noqa: BLE001
        _kernel_failed(exc, "Ozaki fp64 GEMM kernel failed — computed by torch fp64")
        return torch.matmul(ad, bd)


def __getattr__(name):
    if name == "HAS_HIP" or name == "HAS_NKI":
        return has_hip()
    raise AttributeError(name)


# ── op surface ───────────────────────────────────────────────────────────────

_native_ops = None


def get_native_ops() -> dict:
    """The dtype-checked `torch.ops.trnblas.*` ops (registered on first call)."""
    global _native_ops
    if _native_ops is None:
        from . import _native

        _native_ops = _native.OPS
    return _native_ops
