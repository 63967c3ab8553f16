"""Tensor-level wrappers of the C ABI: each takes device tensors, allocates
the output with torch on the operands' device, and launches on torch's
current stream. No routing and no fallback here (see `dispatch.py`): a call
with host tensors, or without the library, raises.
"""

from __future__ import annotations

import os

import torch

from . import _lib
from ._lib import call, ptr, stream_of

# Optional launch probe: when set, called as probe(kernel_name, "begin") and
# probe(kernel_name, "end") right around each C-ABI launch, on the calling
# thread (bench.py records HIP events on the launch stream with it).
_launch_probe = None


def _probed_call(kernel: str, fn: str, *args) -> int:
    probe = _launch_probe
    if probe is None:
        return call(fn, *args)
    probe(kernel, "begin")
    try:
        return call(fn, *args)
    finally:
        probe(kernel, "end")


_gemm_ws: dict = {}


def gemm_workspace(dev: torch.device) -> torch.Tensor:
    """The stream-K workspace of `dev` for torch's current stream there
    (allocated once per stream and reused by every GEMM / SYRK launch on it:
    launches on one stream are ordered, launches on two streams may overlap,
    so each stream has its own)."""
    key = (dev.index if dev.index is not None else torch.cuda.current_device())
    stream = torch._C._cuda_getCurrentRawStream(key)
    ws = _gemm_ws.get((key, stream))
    if ws is None:
        with torch.cuda.device(key):
            n = _lib.load().trnblas_hip_gemm_workspace()
        ws = torch.empty(max(n, 16), dtype=torch.uint8, device=torch.device("cuda", key))
        _gemm_ws[(key, stream)] = ws
    return ws


def _require_device(*ts: torch.Tensor) -> torch.device:
    dev = ts[0].device
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError(f"HIP kernel operands must be on the GPU, got {t.device}")
        if t.device != dev:
            raise ValueError(f"operands on different devices: {dev} and {t.device}")
    return dev


def _mat_layout(X: torch.Tensor):
    """(tensor, trans, ld) describing a 2-D view X without a copy when it is
    row-major (trans=False) or a transposed row-major view (trans=True);
    otherwise a contiguous copy."""
    s0, s1 = X.stride()
    r, c = X.shape
    if s1 == 1 and (s0 >= max(c, 1) or r <= 1):
        return X, False, max(s0, c, 1)
    if s0 == 1 and (s1 >= max(r, 1) or c <= 1):
        return X, True, max(s1, r, 1)
    X = X.contiguous()
    return X, False, max(c, 1)


def _batched_layout(X: torch.Tensor):
    """(tensor, trans, ld, batch_stride) for a 3-D (batch, r, c) view whose
    matrices are row-major or transposed row-major with one batch stride
    (0 = broadcast); else a contiguous copy."""
    b, r, c = X.shape
    sb, s0, s1 = X.stride()
    if b == 1:
        sb = 0
    if s1 == 1 and (s0 >= max(c, 1) or r <= 1):
        return X, False, max(s0, c, 1), sb
    if s0 == 1 and (s1 >= max(r, 1) or c <= 1):
        return X, True, max(s1, r, 1), sb
    X = X.contiguous()
    return X, False, max(c, 1), r * c


# The GEMM / SYRK launcher moves operand panels by LDS DMA only when every
# 16-byte group of an operand lies wholly inside or outside the matrix: a
# 16-byte aligned base, and a leading dimension, batch stride and contiguous
# extent that are multiples of 16 bytes. Other operands run on the
# register-staged kernel: on the MI355X 74 TFLOP/s fp32 at 4095^3 and 8191^3
# (the DMA kernel after packing: 126 and 132) and 81 TFLOP/s bf16 at 4095^3
# (737 after packing). From PACK_MIN_MACS multiply-adds per launch on (by
# element size), such operands are first copied by trnblas_hip_pack_k into
# fresh K-contiguous buffers whose rows are padded with zeros to a multiple
# of 16 bytes (zero products add nothing to any sum; the reference pads its
# kernel operands the same way, nki/dispatch.py:2344-2368) and the product
# takes the DMA kernel. Below it the two pack launches cost more than they
# save (fp32 767^3: 40 us in place, 45 us packed; 1023^3: 52 and 52;
# 1535^3: 126 and 99; bf16 511^3: 29 and 32; 767^3: 38 and 34).
PACK_MIN_MACS = {4: 1 << 30, 2: 1 << 28}

# TRNBLAS_GEMM_RAGGED=0 restores the reference's pad-first path
# (nki/dispatch.py:144-151, read at import as there): every operand the DMA
# kernel cannot read in place is packed and zero-padded first, whatever the
# size; ragged M / N edges stay in the kernel either way.
_RAGGED_ENABLED: bool = os.environ.get("TRNBLAS_GEMM_RAGGED", "1").strip().lower() not in (
    "0", "false", "no", "off",
)  # fmt: skip


def _pack_min_macs(elem_size: int) -> int:
    return PACK_MIN_MACS[elem_size] if _RAGGED_ENABLED else 0


def _dma_ready(t: torch.Tensor, ld: int, stride: int, ext: int, ev: int) -> bool:
    return t.data_ptr() % 16 == 0 and ld % ev == 0 and stride % ev == 0 and ext % ev == 0


def _pack_k(X: torch.Tensor, kp: int) -> torch.Tensor:
    """X (R, K) or (batch, R, K), any strides, copied into a fresh row-major
    (..., R, kp) buffer whose columns K .. kp - 1 are zero (one launch of
    trnblas_hip_pack_k)."""
    R, k = X.shape[-2], X.shape[-1]
    nb, sxb = (X.shape[0], X.stride(0)) if X.dim() == 3 else (1, 0)
    P = torch.empty((*X.shape[:-1], kp), dtype=X.dtype, device=X.device)
    call(
        "trnblas_hip_pack_k", _lib.DTYPE_CODES[X.dtype], R, k, ptr(X), X.stride(-2),
        X.stride(-1), sxb, ptr(P), kp, R * kp, nb, stream_of(X.device),
    )  # fmt: skip
    return P


def _packed_operands(A, B, a, ta, lda, sa, b, tb, ldb, sb, M, N, K, nb):
    """The C-ABI operand arguments of A (M, K) and B (K, N) (3-D: batched,
    batch 1 broadcast): (a, ta, lda, sa, b, tb, ldb, sb, K) as laid out, or
    with the operands the DMA kernel cannot read packed K-contiguous (and K
    padded when it is not a multiple of 16 bytes)."""
    ev = 16 // A.element_size()
    if nb * M * N * K < _pack_min_macs(A.element_size()) or M == 0 or N == 0 or K == 0:
        return a, ta, lda, sa, b, tb, ldb, sb, K
    a_ok = _dma_ready(a, lda, sa, M if ta else K, ev)
    b_ok = _dma_ready(b, ldb, sb, K if tb else N, ev)
    kp = -(-K // ev) * ev
    if a_ok and b_ok:
        return a, ta, lda, sa, b, tb, ldb, sb, K
    if kp != K or not a_ok:
        pa = _pack_k(A, kp)
        a, ta, lda, sa = pa, False, kp, (M * kp if pa.dim() == 3 and pa.shape[0] > 1 else 0)
    if kp != K or not b_ok:
        pb = _pack_k(B.transpose(-1, -2), kp)
        b, tb, ldb, sb = pb, True, kp, (N * kp if pb.dim() == 3 and pb.shape[0] > 1 else 0)
    return a, ta, lda, sa, b, tb, ldb, sb, kp


def _packed_syrk_operand(A, trans, a, t, lda, n, k):
    """SYRK's (a, t, lda, k) for op(A) (n, k): as laid out, or packed
    K-contiguous with k padded to a multiple of 16 bytes (see _packed_operands)."""
    ev = 16 // A.element_size()
    if n * n * k < _pack_min_macs(A.element_size()) or n == 0 or k == 0 or _dma_ready(a, lda, 0, n if t else k, ev):
        return a, t, lda, k
    kp = -(-k // ev) * ev
    return _pack_k(A.t() if trans else A, kp), False, kp, kp


def gemm(
    A: torch.Tensor,
    B: torch.Tensor,
    alpha: float = 1.0,
    beta: float = 0.0,
    C: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """alpha * A @ B + beta * C for device A (M, K), B (K, N) (or batched
    (b, M, K), (b, K, N) with equal or broadcast batch), one launch. Transposed
    views are read in place. Returns a fresh (M, N) / (b, M, N) tensor in
    A's dtype; C (same shape, or broadcast over the batch) is never written.
    out (2-D only): an (M, N) view with unit column stride to write instead,
    which may be C itself (an in-place update; each element of C is read
    and written by the same thread) but must not overlap A or B."""
    dev = _require_device(A, B, *(() if C is None else (C,)))
    if A.dtype != B.dtype or (C is not None and C.dtype != A.dtype):
        raise TypeError(f"gemm: mixed dtypes {A.dtype}, {B.dtype}")
    code = _lib.DTYPE_CODES.get(A.dtype)
    if code is None:
        raise TypeError(f"gemm: dtype {A.dtype} not supported by the HIP kernel")
    if A.dim() == 2 and B.dim() == 2:
        M, K = A.shape
        K2, N = B.shape
        if K != K2:
            raise ValueError(f"gemm: inner dimensions differ: {tuple(A.shape)} @ {tuple(B.shape)}")
        a, ta, lda = _mat_layout(A)
        b, tb, ldb = _mat_layout(B)
        a, ta, lda, _, b, tb, ldb, _, K = _packed_operands(
            A, B, a, ta, lda, 0, b, tb, ldb, 0, M, N, K, 1
        )
        if out is None:
            D, ldd = torch.empty((M, N), dtype=A.dtype, device=dev), N
        else:
            if tuple(out.shape) != (M, N) or out.dtype != A.dtype or out.device != dev:
                raise ValueError(f"gemm: out must be ({M}, {N}) {A.dtype} on {dev}")
            if M and N and (out.stride(1) != 1 or out.stride(0) < N):
                raise ValueError("gemm: out needs unit column stride and a row stride >= N")
            D, ldd = out, max(out.stride(0), N)
        ws = gemm_workspace(dev)
        c, ldc = None, N
        if beta != 0.0 and C is not None:
            c = C if tuple(C.shape) == (M, N) else C.expand(M, N)
            if c.stride(1) != 1 or c.stride(0) < N:
                c = c.contiguous()
            ldc = c.stride(0)
        _probed_call(
            "gemm", "trnblas_hip_gemm", code, int(ta), int(tb), M, N, K, float(alpha),
            ptr(a), lda, 0, ptr(b), ldb, 0, float(beta) if c is not None else 0.0,
            ptr(c), ldc, 0, ptr(D), ldd, 0, 1, ptr(ws), ws.numel(), stream_of(dev),
        )  # fmt: skip
        return D
    if out is not None:
        raise ValueError("gemm: out is supported for 2-D operands only")
    if A.dim() != 3 or B.dim() != 3:
        raise ValueError("gemm: operands must both be 2-D or both 3-D")
    bA, M, K = A.shape
    bB, K2, N = B.shape
    if K != K2:
        raise ValueError(f"gemm: inner dimensions differ: {tuple(A.shape)} @ {tuple(B.shape)}")
    nb = max(bA, bB)
    if bA not in (1, nb) or bB not in (1, nb):
        raise ValueError(f"gemm: batch sizes {bA} and {bB} do not broadcast")
    a, ta, lda, sa = _batched_layout(A)
    b, tb, ldb, sb = _batched_layout(B)
    a, ta, lda, sa, b, tb, ldb, sb, K = _packed_operands(
        A, B, a, ta, lda, sa, b, tb, ldb, sb, M, N, K, nb
    )
    D = torch.empty((nb, M, N), dtype=A.dtype, device=dev)
    ws = gemm_workspace(dev)
    c, ldc, sc = None, N, 0
    if beta != 0.0 and C is not None:
        c = C.expand(nb, M, N)
        if c.stride(2) != 1 or c.stride(1) < N:
            c = c.contiguous()
        ldc, sc = c.stride(1), (0 if nb == 1 else c.stride(0))
    _probed_call(
        "gemm", "trnblas_hip_gemm", code, int(ta), int(tb), M, N, K, float(alpha),
        ptr(a), lda, sa, ptr(b), ldb, sb, float(beta) if c is not None else 0.0,
        ptr(c), ldc, sc, ptr(D), N, M * N, nb, ptr(ws), ws.numel(), stream_of(dev),
    )  # fmt: skip
    return D


def syrk(
    A: torch.Tensor,
    alpha: float = 1.0,
    beta: float = 0.0,
    C: torch.Tensor | None = None,
    trans: bool = False,
    uplo: str = "lower",
) -> torch.Tensor:
    """alpha * op(A) op(A)^T + beta * sym_uplo(C), full symmetric (n, n),
    computing only the lower triangle of the product. op(A) = A (n, k), or
    A^T for trans (A (k, n))."""
    dev = _require_device(A, *(() if C is None else (C,)))
    code = _lib.DTYPE_CODES.get(A.dtype)
    if code is None:
        raise TypeError(f"syrk: dtype {A.dtype} not supported by the HIP kernel")
    a, t, lda = _mat_layout(A)
    t = t != bool(trans)  # a transposed view flips the layout flag
    n = A.shape[1] if trans else A.shape[0]
    k = A.shape[0] if trans else A.shape[1]
    a, t, lda, k = _packed_syrk_operand(A, trans, a, t, lda, n, k)
    D = torch.empty((n, n), dtype=A.dtype, device=dev)
    ws = gemm_workspace(dev)
    c, ldc = None, n
    if beta != 0.0 and C is not None:
        if C.dtype != A.dtype:
            raise TypeError("syrk: C dtype differs from A")
        c = C if (C.stride(1) == 1 and C.stride(0) >= n) else C.contiguous()
        ldc = c.stride(0)
    _probed_call(
        "syrk", "trnblas_hip_syrk", code, 1 if uplo == "upper" else 0, int(t), n, k, float(alpha),
        ptr(a), lda, float(beta) if c is not None else 0.0, ptr(c), ldc, ptr(D), n,
        ptr(ws), ws.numel(), stream_of(dev),
    )  # fmt: skip
    return D


_side_streams: dict = {}


def _side_stream(dev: torch.device) -> "torch.cuda.Stream":
    """A second stream of `dev` (default priority) for small host reads that
    must not wait behind the main stream's later work."""
    s = _side_streams.get(dev.index)
    if s is None:
        s = _side_streams[dev.index] = torch.cuda.Stream(dev)
    return s


def syrk_checked(
    A: torch.Tensor,
    alpha: float,
    beta: float,
    C: torch.Tensor,
    trans: bool = False,
    uplo: str = "upper",
) -> tuple[torch.Tensor, bool, bool]:
    """`syrk` with beta != 0 and the triangle rule of an n x n C decided on
    the device: returns (D, uplo triangle has an off-diagonal nonzero, the
    other triangle has one). The triangle check, then the SYRK reading its
    flags, run back to back on the current stream; the flags reach the host
    over a side stream, so the host waits for the check only, not for the
    product."""
    dev = _require_device(A, C)
    code = _lib.DTYPE_CODES.get(A.dtype)
    if code is None:
        raise TypeError(f"syrk: dtype {A.dtype} not supported by the HIP kernel")
    if C.dtype != A.dtype:
        raise TypeError("syrk: C dtype differs from A")
    a, t, lda = _mat_layout(A)
    t = t != bool(trans)
    n = A.shape[1] if trans else A.shape[0]
    k = A.shape[0] if trans else A.shape[1]
    a, t, lda, k = _packed_syrk_operand(A, trans, a, t, lda, n, k)
    if tuple(C.shape) != (n, n):
        raise ValueError(f"syrk: C must be {n} x {n}, got {tuple(C.shape)}")
    c = C if (C.stride(1) == 1 and C.stride(0) >= n) else C.contiguous()
    ldc = c.stride(0)
    D = torch.empty((n, n), dtype=A.dtype, device=dev)
    ws = gemm_workspace(dev)
    flags = torch.empty(2, dtype=torch.int32, device=dev)
    main = torch.cuda.current_stream(dev)
    call("trnblas_hip_triangle_nonzero", code, n, ptr(c), ldc, ptr(flags), stream_of(dev))
    checked = torch.cuda.Event()
    checked.record(main)
    side = _side_stream(dev)
    side.wait_event(checked)
    host = torch.empty(2, dtype=torch.int32, pin_memory=True)
    with torch.cuda.stream(side):
        host.copy_(flags, non_blocking=True)
        landed = torch.cuda.Event()
        landed.record(side)
    flags.record_stream(side)
    _probed_call(
        "syrk", "trnblas_hip_syrk_flagged", code, 1 if uplo == "upper" else 0, int(t), n, k,
        float(alpha), ptr(a), lda, float(beta), ptr(c), ldc, ptr(D), n, ptr(flags),
        ptr(ws), ws.numel(), stream_of(dev),
    )  # fmt: skip
    landed.synchronize()
    up, lo = (bool(v) for v in host.tolist())
    mine, theirs = (up, lo) if uplo == "upper" else (lo, up)
    return D, mine, theirs


# ── DF-MP2 pair energy ───────────────────────────────────────────────────────


def _pe_operand(X: torch.Tensor) -> torch.Tensor:
    """fp32 (n, nvir, naux) with the aux index contiguous (a view if it is)."""
    if X.dtype != torch.float32:
        raise TypeError(f"pair energy kernel takes float32 amplitudes, got {X.dtype}")
    if X.stride(-1) != 1 or (X.shape[1] > 1 and X.stride(1) < X.shape[2]):
        X = X.contiguous()
    return X


PAIR_ENERGY_MATH = ("fp32", "bf16x6", "fp16x3")


_PE_ENTRY = {
    "fp32": "trnblas_hip_pair_energy",
    "bf16x6": "trnblas_hip_pair_energy_bf16x6",
    "fp16x3": "trnblas_hip_pair_energy_fp16x3",
}


def pair_energy_math() -> str:
    """Arithmetic of the fused pair-energy kernel: TRNBLAS_PAIR_ENERGY_MATH =
    "fp16x3" (default, the fastest: f16 MFMA on two-piece splits of
    row-scaled operands, three products, fp32 slice sums), "bf16x6" (bf16
    MFMA on three-piece splits, six products; the most accurate) or "fp32"
    (fp32 MFMA).

    Accuracy per product x y: fp32 MFMA and bf16x6 are within about 2^-22 of
    x y; fp16x3 keeps 22 significand bits per operand and drops lo_x lo_y, so
    within 3 2^-22 (about 4x fp32's), and an entry more than 2^28 below its
    row's largest entry becomes an fp16 subnormal with an absolute error of
    at most 2^-39 of that maximum rather than a relative one. On energies
    (sums dominated by the large entries) all three meet rel 1e-6 against
    fp64 (C3: fp16x3 2.3e-9, fp32 2.3e-9, bf16x6 1.3e-10); callers that need
    fp32-class accuracy product by product choose "bf16x6" or "fp32"."""
    return _check_math(os.environ.get("TRNBLAS_PAIR_ENERGY_MATH", "fp16x3").strip().lower())


def _check_math(math: str | None) -> str:
    if math is None:
        return pair_energy_math()
    if math not in PAIR_ENERGY_MATH:
        raise ValueError(f"pair energy math must be one of {PAIR_ENERGY_MATH}; got {math!r}")
    return math


def pair_energy_sym(B: torch.Tensor, eps_occ: torch.Tensor, eps_vir: torch.Tensor, math: str | None = None):
    """E = sum_{i,j} e_ij over all ordered pairs, evaluated as the i <= j walk
    (weights 1 / 2) in one launch. B (nocc, nvir, naux) fp32 on the GPU.
    math: "fp32" (fp32 MFMA), "bf16x6" (each fp32 operand split into three
    bf16 pieces by a first pass; six bf16 MFMA products per fp32 product),
    "fp16x3" (each row scaled by a power of two and split into two fp16
    pieces; three f16 MFMA products per fp32 product) or None
    (pair_energy_math()). Returns a 0-d float64 device tensor."""
    dev = _require_device(B, eps_occ, eps_vir)
    math = _check_math(math)
    B = _pe_operand(B)
    nocc, nvir, naux = B.shape
    eo = eps_occ.to(torch.float32).contiguous()
    ev = eps_vir.to(torch.float32).contiguous()
    total = torch.empty((), dtype=torch.float64, device=dev)
    npairs = nocc * (nocc + 1) // 2
    ld_occ = B.stride(0) if nocc > 1 else nvir * naux
    _pe_launch(
        math, dev, nvir, naux, B, nocc, ld_occ, B, 0, ld_occ, B.stride(1) if nvir > 1 else naux,
        eo, eo, ev, nocc, npairs, None, None, None, total, probed=True,
    )  # fmt: skip
    return total


def _pe_launch(math, dev, nvir, naux, Bi, ni, ldi, Bj, nj, ldj, ld_vir, ei, ej, ev, nocc, npairs,
               pi, pj, out_pairs, out_total, probed=False):
    """One pair-energy launch with its workspace. ni / nj: rows of Bi / Bj
    (nj == 0: Bj is Bi), used by the split entry points for their planes."""
    lib = _lib.load()
    if math in ("bf16x6", "fp16x3"):
        ws = getattr(lib, _PE_ENTRY[math] + "_workspace")(nvir, naux, npairs, ni, nj)
        head = (nvir, naux, ptr(Bi), ni, ldi, ptr(Bj), nj, ldj, ld_vir)
    else:
        ws = lib.trnblas_hip_pair_energy_workspace(nvir, npairs)
        head = (nvir, naux, ptr(Bi), ldi, ptr(Bj), ldj, ld_vir)
    work = torch.empty(max(ws, 8), dtype=torch.uint8, device=dev)
    args = head + (ptr(ei), ptr(ej), ptr(ev), nocc, npairs, ptr(pi), ptr(pj), None,
                   ptr(out_pairs), ptr(out_total), ptr(work), work.numel(), stream_of(dev))
    if probed:
        _probed_call("pair_energy", _PE_ENTRY[math], *args)
    else:
        call(_PE_ENTRY[math], *args)


def pair_energies(
    Bi: torch.Tensor,
    Bj: torch.Tensor,
    eps_i: torch.Tensor,
    eps_j: torch.Tensor,
    eps_vir: torch.Tensor,
    pair_i: torch.Tensor,
    pair_j: torch.Tensor,
    math: str | None = None,
) -> torch.Tensor:
    """Unweighted e_p for the pairs (pair_i[p], pair_j[p]), with T = Bi[i]
    Bj[j]^T. Bi (ni, nvir, naux), Bj (nj, nvir, naux) fp32; returns float64
    (npairs,) on the device. math as in pair_energy_sym."""
    dev = _require_device(Bi, Bj, eps_i, eps_j, eps_vir)
    math = _check_math(math)
    Bi, Bj = _pe_operand(Bi), _pe_operand(Bj)
    if Bi.shape[1:] != Bj.shape[1:]:
        raise ValueError(f"pair operands differ: {tuple(Bi.shape)} vs {tuple(Bj.shape)}")
    if Bi.stride(1) != Bj.stride(1):
        Bi, Bj = Bi.contiguous(), Bj.contiguous()
    _, nvir, naux = Bi.shape
    pi = pair_i.to(device=dev, dtype=torch.int32).contiguous()
    pj = pair_j.to(device=dev, dtype=torch.int32).contiguous()
    npairs = pi.numel()
    out = torch.empty(npairs, dtype=torch.float64, device=dev)
    if npairs == 0:
        return out
    ei = eps_i.to(torch.float32).contiguous()
    ej = eps_j.to(torch.float32).contiguous()
    ev = eps_vir.to(torch.float32).contiguous()
    ld_vir = Bi.stride(1) if nvir > 1 else naux
    same = Bj.data_ptr() == Bi.data_ptr() and Bj.shape == Bi.shape and Bj.stride() == Bi.stride()
    _pe_launch(
        math, dev, nvir, naux, Bi, Bi.shape[0], Bi.stride(0), Bj, 0 if same else Bj.shape[0],
        Bj.stride(0), ld_vir, ei, ej, ev, 0, npairs, pi, pj, out, None,
    )  # fmt: skip
    return out


def mp2_energy_pairs(T_flat, eps_occ_chunk, eps_occ_full, eps_vir) -> torch.Tensor:
    """Per-pair MP2 energies (ic * nocc,) float64 of a precomputed T_flat
    (ic * nvir, nocc * nvir) fp32 (row stride >= nocc * nvir)."""
    dev = _require_device(T_flat, eps_occ_chunk, eps_occ_full, eps_vir)
    if T_flat.dtype != torch.float32:
        raise TypeError("mp2_energy kernel takes float32 T_flat")
    if T_flat.stride(1) != 1:
        T_flat = T_flat.contiguous()
    ic, nocc, nvir = eps_occ_chunk.numel(), eps_occ_full.numel(), eps_vir.numel()
    out = torch.empty(ic * nocc, dtype=torch.float64, device=dev)
    f32 = torch.float32
    eoc = eps_occ_chunk.to(f32).contiguous()
    eof = eps_occ_full.to(f32).contiguous()
    ev = eps_vir.to(f32).contiguous()
    call(
        "trnblas_hip_mp2_energy", ic, nocc, nvir, ptr(T_flat), T_flat.stride(0) if ic else 1,
        ptr(eoc), ptr(eof), ptr(ev), ptr(out), stream_of(dev),
    )  # fmt: skip
    return out


# ── metric stage ─────────────────────────────────────────────────────────────

def _dgemm_operand(X: torch.Tensor, is_a: bool):
    """(tensor, trans, ld, batch stride) of a 3-D fp64 operand for
    trnblas_hip_dgemm: a row-major or transposed row-major view as is, when
    its base is 16-byte aligned and its leading dimension, batch stride and
    contiguous extent are even; otherwise a K-contiguous copy (K is even
    here: dgemm pads an odd K)."""
    t, tr, ld, sb = _batched_layout(X)
    ext = t.shape[1] if tr else t.shape[2]
    if ptr(t) % 16 == 0 and ld % 2 == 0 and sb % 2 == 0 and ext % 2 == 0:
        return t, tr, ld, sb
    c = X.contiguous() if is_a else X.mT.contiguous()  # A (b, M, K); B stored (b, N, K)
    return c, not is_a, c.shape[2], (0 if c.shape[0] == 1 else c.shape[1] * c.shape[2])


def dgemm(
    A: torch.Tensor,
    B: torch.Tensor,
    alpha: float = 1.0,
    beta: float = 0.0,
    C: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    lower: bool = False,
    tri: int = 0,
) -> torch.Tensor:
    """fp64 alpha * A @ B + beta * C on the fp64 MFMA (trnblas_hip_dgemm):
    A (M, K), B (K, N), or batched (b, M, K) @ (b, K, N) (a batch of 1
    broadcasts). Transposed views are read in place. out: the (M, N) /
    (b, M, N) tensor to write (unit column stride, row stride >= N), which
    may be C itself; otherwise a fresh tensor. lower (2-D, M == N): only the
    elements m >= n are computed and written. tri: _lib.TRI_* bits of
    triangular operands whose zero blocks the kernel skips (their other
    triangle must hold zeros)."""
    dev = _require_device(A, B, *(() if C is None else (C,)), *(() if out is None else (out,)))
    for X in (A, B) + (() if C is None else (C,)) + (() if out is None else (out,)):
        if X.dtype != torch.float64:
            raise TypeError(f"dgemm: float64 operands only, got {X.dtype}")
    two = A.dim() == 2 and B.dim() == 2
    if not two and not (A.dim() == 3 and B.dim() == 3):
        raise ValueError("dgemm: operands must both be 2-D or both 3-D")
    M, K = A.shape[-2:]
    K2, N = B.shape[-2:]
    if K != K2:
        raise ValueError(f"dgemm: inner dimensions differ: {tuple(A.shape)} @ {tuple(B.shape)}")
    nb = 1 if two else max(A.shape[0], B.shape[0])
    if not two and (A.shape[0] not in (1, nb) or B.shape[0] not in (1, nb)):
        raise ValueError(f"dgemm: batch sizes {A.shape[0]} and {B.shape[0]} do not broadcast")
    if lower and (not two or M != N):
        raise ValueError("dgemm: lower needs a square 2-D product")
    shape = (M, N) if two else (nb, M, N)
    if out is None:
        out = torch.empty(shape, dtype=torch.float64, device=dev)
    if tuple(out.shape) != shape:
        raise ValueError(f"dgemm: out must be {shape}")
    o3 = out if out.dim() == 3 else out.unsqueeze(0)
    if M and N and (o3.stride(2) != 1 or o3.stride(1) < N):
        raise ValueError("dgemm: out needs unit column stride and a row stride >= N")
    ldd, sd = max(o3.stride(1), N), (o3.stride(0) if nb > 1 else 0)
    A3 = A if A.dim() == 3 else A.unsqueeze(0)
    B3 = B if B.dim() == 3 else B.unsqueeze(0)
    if K % 2:  # a zero term makes K even (16-byte groups along K)
        A3 = torch.nn.functional.pad(A3, (0, 1))
        B3 = torch.nn.functional.pad(B3, (0, 0, 0, 1))
        K += 1
    a, ta, lda, sa = _dgemm_operand(A3, True)
    b, tb, ldb, sb = _dgemm_operand(B3, False)
    c, ldc, sc = None, N, 0
    if beta != 0.0 and C is not None:
        c3 = (C if C.dim() == 3 else C.unsqueeze(0)).expand(nb, M, N)
        if c3.stride(2) != 1 or c3.stride(1) < N:
            c3 = c3.contiguous()
        c, ldc, sc = c3, c3.stride(1), (c3.stride(0) if nb > 1 else 0)
    _probed_call(
        "dgemm", "trnblas_hip_dgemm", int(ta), int(tb), M, N, K, float(alpha),
        ptr(a), lda, sa, ptr(b), ldb, sb, float(beta) if c is not None else 0.0,
        ptr(c), ldc, sc, ptr(o3), ldd, sd, nb, int(lower), int(tri), stream_of(dev),
    )  # fmt: skip
    return out


TRI_NB = 128  # block of trnblas_hip_tri_inv_blocks


def tri_inv_blocks(T: torch.Tensor, upper: bool, unit: bool = False) -> torch.Tensor:
    """Inverses of the 128 x 128 diagonal blocks of the triangular (n, n)
    device matrix T (float32 or float64, any strides; only the `upper` /
    lower triangle is read, the diagonal taken as ones when unit): a
    (ceil(n / 128), 128, 128) tensor of T's dtype, block b the inverse of
    T[128 b:128 b + 128, 128 b:128 b + 128] padded with the identity."""
    dev = _require_device(T)
    if T.dim() != 2 or T.shape[0] != T.shape[1]:
        raise ValueError(f"tri_inv_blocks: T must be square, got {tuple(T.shape)}")
    codes = {torch.float32: _lib.F32, torch.float64: _lib.F64}
    if T.dtype not in codes:
        raise TypeError(f"tri_inv_blocks: float32 / float64 only, got {T.dtype}")
    n = T.shape[0]
    nblk = -(-n // TRI_NB)
    D = torch.empty((nblk, TRI_NB, TRI_NB), dtype=T.dtype, device=dev)
    if n:
        sr, sc = T.stride()
        call(
            "trnblas_hip_tri_inv_blocks", codes[T.dtype], n, int(bool(upper)), int(bool(unit)),
            ptr(T), max(sr, 1), max(sc, 1), ptr(D), stream_of(dev),
        )  # fmt: skip
    return D


def metric_inv_half(J: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(X, info) for the SPD (n, n) float64 device matrix J (lower triangle
    read): X = L^-T with J = L L^T, exactly upper triangular, from the
    native driver trnblas_hip_metric_inv_half (blocked Cholesky, block
    inverse, transpose; one call); info (int32 device tensor of one element)
    holds the order of the first leading minor that is not positive
    definite, else 0."""
    dev = _require_device(J)
    if J.dtype != torch.float64 or J.dim() != 2 or J.shape[0] != J.shape[1]:
        raise ValueError("metric_inv_half: J must be a square float64 matrix")
    n = J.shape[0]
    X = torch.empty((n, n), dtype=torch.float64, device=dev)
    info = torch.zeros(1, dtype=torch.int32, device=dev)
    if n == 0:
        return X, info
    if J.stride(1) != 1 or J.stride(0) < n:
        J = J.contiguous()
    lib = _lib.load()
    with torch.cuda.device(dev):
        ws = torch.empty(lib.trnblas_hip_metric_inv_half_workspace(n), dtype=torch.uint8, device=dev)
        _probed_call(
            "metric_inv_half", "trnblas_hip_metric_inv_half", n, ptr(J), J.stride(0), ptr(X), n,
            ptr(info), ptr(ws), ws.numel(), stream_of(dev),
        )  # fmt: skip
    return X, info


def trsm(T: torch.Tensor, B: torch.Tensor, upper: bool, unit: bool, alpha: float,
         out: torch.Tensor) -> torch.Tensor:
    """T X = alpha B for the triangular (n, n) device matrix T (`upper` /
    lower triangle read; unit: its diagonal taken as ones) and B (n, m),
    float32 or float64, any strides, into out (n, m, any positive strides,
    e.g. the transposed view of a right solve's result), through the native
    driver trnblas_hip_trsm. Returns out."""
    dev = _require_device(T, B, out)
    codes = {torch.float32: _lib.F32, torch.float64: _lib.F64}
    if T.dtype not in codes or B.dtype != T.dtype or out.dtype != T.dtype:
        raise TypeError(f"trsm: float32 / float64 operands of one dtype, got {T.dtype}, {B.dtype}")
    n, m = B.shape
    if tuple(T.shape) != (n, n) or tuple(out.shape) != (n, m):
        raise ValueError(f"trsm: T {tuple(T.shape)}, B {tuple(B.shape)}, out {tuple(out.shape)}")
    if n == 0 or m == 0:
        return out
    lib = _lib.load()
    code = codes[T.dtype]

    def st(x):
        return max(x.stride(0), 1), max(x.stride(1), 1)

    with torch.cuda.device(dev):
        ws = torch.empty(lib.trnblas_hip_trsm_workspace(code, n, m), dtype=torch.uint8, device=dev)
        _probed_call(
            "trsm", "trnblas_hip_trsm", code, n, m, int(bool(upper)), int(bool(unit)), float(alpha),
            ptr(T), *st(T), ptr(B), *st(B), ptr(out), *st(out), ptr(ws), ws.numel(), stream_of(dev),
        )  # fmt: skip
    return out


CHOL_NB = 128  # largest diagonal block of trnblas_hip_chol_block


def chol_block(A: torch.Tensor, Linv: torch.Tensor, info: torch.Tensor, offset: int) -> None:
    """One diagonal block (nb <= 128) of the blocked metric Cholesky, in
    place on the device: A's lower triangle becomes L (A = L L^T), Linv
    becomes L^-1 (lower, zeros above), and info[0] becomes offset + the first
    non-positive pivot (1-based) unless it is already nonzero. A and Linv are
    (nb, nb) float64 views with unit column stride; info is int32."""
    dev = _require_device(A, Linv, info)
    if A.dtype != torch.float64 or Linv.dtype != torch.float64 or info.dtype != torch.int32:
        raise TypeError("chol_block takes float64 A / Linv and an int32 info")
    nb = A.shape[0]
    if A.dim() != 2 or A.shape[1] != nb or tuple(Linv.shape) != (nb, nb):
        raise ValueError("chol_block: A and Linv must both be (nb, nb)")
    if nb > CHOL_NB:
        raise ValueError(f"chol_block: nb {nb} > {CHOL_NB}")
    if nb and (A.stride(1) != 1 or Linv.stride(1) != 1):
        raise ValueError("chol_block: A and Linv need unit column stride")
    call(
        "trnblas_hip_chol_block", nb, ptr(A), A.stride(0) if nb else 1, ptr(Linv),
        Linv.stride(0) if nb else 1, ptr(info), offset, stream_of(dev),
    )  # fmt: skip


# ── Ozaki ────────────────────────────────────────────────────────────────────

OZ_TILE = 128  # K padding of the digit stacks (ozaki.TILE_K)
OZ_ROW_PAD = 128  # row padding of the digit stacks (tile of the slice GEMM)


def _round_up(n: int, m: int) -> int:
    return -(-n // m) * m


def ozaki_split(X: torch.Tensor, slices: int, per: str, interleaved: bool = False):
    """Digits and exponents of a device fp64 matrix X (R, C).

    per="row": digits (k, Rp, Cp) int8 with digit[s, r, c] (K = C contiguous);
    per="col": digits (k, Cp, Rp) int8 with digit[s, c, r] (K = R contiguous,
    the column split written transposed). Exponents int32 (R,) / (C,).
    interleaved: digits (rows, Kp * k) instead, the k slices of each 32-wide
    K chunk of a row side by side (the fast GEMM's operand layout).
    Returns (digits, exps, nonfinite) where `nonfinite` is a 0-d int32 device
    flag (the digits are undefined when it is set)."""
    dev = _require_device(X)
    if X.dtype != torch.float64:
        raise TypeError("ozaki_split takes float64")
    if X.stride(-1) != 1:
        X = X.contiguous()
    R, C = X.shape
    per_row = per == "row"
    rows, cols = (R, C) if per_row else (C, R)
    rp, cp = _round_up(max(rows, 1), OZ_ROW_PAD), _round_up(max(cols, 1), OZ_TILE)
    # the split writes every digit of the R x C matrix: only padding needs zeros
    alloc = torch.empty if (rp, cp) == (rows, cols) else torch.zeros
    if interleaved:
        digits = alloc((rp, cp * slices), dtype=torch.int8, device=dev)
        flags, ld_digit, ld_slice = int(per_row) | 2, cp * slices, 0
    else:
        digits = alloc((slices, rp, cp), dtype=torch.int8, device=dev)
        flags, ld_digit, ld_slice = int(per_row), cp, rp * cp
    exps = torch.empty(rows, dtype=torch.int32, device=dev)
    scratch = torch.zeros(2, dtype=torch.int32, device=dev)
    call(
        "trnblas_hip_ozaki_split", flags, R, C, ptr(X), X.stride(0) if R else 1,
        slices, ptr(digits), ld_digit, ld_slice, ptr(exps), ptr(scratch), stream_of(dev),
    )  # fmt: skip
    return digits, exps, scratch[1]


def ozaki_gemm(dA, eA, dB, eB, M: int, N: int, slices: int, kb: int | None = None,
               out: torch.Tensor | None = None, transpose_out: bool = False,
               fast: bool = False) -> torch.Tensor:
    """fp64 C (M, N) from digit stacks dA (k, >=M, Kp), dB (k, >=N, Kp)
    (K-contiguous) and their exponents: the bit-exact schedule (fast=False,
    K blocks of kb) or the fast one (int32 diagonals, fp64 recombination; kb
    unused). 2-D dA / dB are interleaved digits (ozaki_split(interleaved=True),
    fast only). With transpose_out, writes C^T into `out` (N, M)
    instead."""
    dev = _require_device(dA, dB, eA, eB)
    interleaved = dA.dim() == 2
    if interleaved:
        if not fast or dB.dim() != 2:
            raise ValueError("interleaved digits are for the fast schedule, both operands")
        k, Kp = slices, dA.shape[1] // slices
        mode, lda_s, ldb_s = 2, 0, 0
    else:
        k, _, Kp = dA.shape
        mode, lda_s, ldb_s = (1 if fast else 0), dA.stride(0), dB.stride(0)
    kb = Kp if kb is None else kb
    if out is None:
        out = torch.empty((N, M) if transpose_out else (M, N), dtype=torch.float64, device=dev)
    if transpose_out:
        ldc_m, ldc_n = out.stride(1), out.stride(0)
    else:
        ldc_m, ldc_n = out.stride(0), out.stride(1)
    lda, ldb = (dA.stride(0), dB.stride(0)) if interleaved else (dA.stride(1), dB.stride(1))
    _probed_call(
        "ozaki_gemm", "trnblas_hip_ozaki_gemm", mode, slices, M, N, Kp, kb, ptr(dA), lda,
        lda_s, ptr(dB), ldb, ldb_s, ptr(eA), ptr(eB), ptr(out), ldc_m, ldc_n, stream_of(dev),
    )  # fmt: skip
    return out


CRT_KP = 64  # K padding of the residue operands (the CRT GEMM's k-step)


def crt_moduli(slices: int, K: int) -> int:
    """Moduli the scheme-II product of inner dimension K needs at `slices`
    (trnblas_hip_crt_moduli; host arithmetic, no device call)."""
    return call("trnblas_hip_crt_moduli", slices, K)


def crt_split(X: torch.Tensor, slices: int, nmod: int, per: str, kp: int):
    """Exponents and int8 residues of a device fp64 matrix X (R, C) for the
    first nmod moduli: per="row" -> residues of the rows (K = C), per="col"
    -> of the columns (K = R). The residues are blocked, 16 operand rows x
    64 K values per contiguous KiB: a (nmod, ceil(rows / 16), kp / 64, 16, 64)
    tensor, element (t, r, k) at [t, r // 16, k // 64, r % 16, k % 64].
    Returns (residues, exps, nonfinite) with `nonfinite` a 0-d device flag."""
    dev = _require_device(X)
    if X.dtype != torch.float64:
        raise TypeError("crt_split takes float64")
    if X.stride(-1) != 1:
        X = X.contiguous()
    R, C = X.shape
    rows = R if per == "row" else C
    rb = -(-rows // 16)
    res = torch.empty((nmod, rb, kp // 64, 16, 64), dtype=torch.int8, device=dev)
    exps = torch.empty(rows, dtype=torch.int32, device=dev)
    flags = torch.zeros(2, dtype=torch.int32, device=dev)
    _probed_call(
        "crt_split", "trnblas_hip_crt_split", int(per == "row"), R, C, ptr(X), X.stride(0),
        slices, nmod, kp, ptr(res), res.stride(0), ptr(exps), ptr(flags), stream_of(dev),
    )  # fmt: skip
    return res, exps, flags[1]


def crt_unblock(res: torch.Tensor) -> torch.Tensor:
    """(nmod, rows16, kp) view-order copy of blocked residues (tests)."""
    n, rb, kc, _, _ = res.shape
    return res.permute(0, 1, 3, 2, 4).reshape(n, rb * 16, kc * 64)


def crt_gemm(RA: torch.Tensor, RB: torch.Tensor, M: int, N: int) -> torch.Tensor:
    """Product residues P_t = RA_t RB_t^T mod m_t from blocked residues
    (crt_split), 32 x 32 blocked (see trnblas_hip_crt_gemm):
    (nmod, ceil(M/32) ceil(N/32) 1024) int8."""
    dev = _require_device(RA, RB)
    nmod, kp = RA.shape[0], RA.shape[2] * 64
    plane = -(-M // 32) * -(-N // 32) * 1024
    P = torch.empty((nmod, plane), dtype=torch.int8, device=dev)
    _probed_call(
        "crt_gemm", "trnblas_hip_crt_gemm", nmod, M, N, kp, ptr(RA), RA.stride(0), ptr(RB),
        RB.stride(0), ptr(P), plane, stream_of(dev),
    )  # fmt: skip
    return P


def crt_combine(P: torch.Tensor, eA: torch.Tensor, eB: torch.Tensor, M: int, N: int, slices: int,
                out: torch.Tensor | None = None, transpose_out: bool = False) -> torch.Tensor:
    """fp64 C (M, N) (or C^T into `out` (N, M) with transpose_out) from the
    product residue planes and the operand exponents."""
    dev = _require_device(P, eA, eB)
    if out is None:
        out = torch.empty((N, M) if transpose_out else (M, N), dtype=torch.float64, device=dev)
    ldc_m, ldc_n = (out.stride(1), out.stride(0)) if transpose_out else (out.stride(0), out.stride(1))
    _probed_call(
        "crt_combine", "trnblas_hip_crt_combine", slices, P.shape[0], M, N, ptr(P), P.stride(0),
        ptr(eA), ptr(eB), ptr(out), ldc_m, ldc_n, stream_of(dev),
    )  # fmt: skip
    return out


def ozaki_hilo(dA, dB, M: int, N: int, slices: int) -> torch.Tensor:
    """Raw (2, M, N) fp32 (hi, lo) of the slice GEMM (one K block)."""
    dev = _require_device(dA, dB)
    Kp = dA.shape[2]
    hilo = torch.empty((2, M, N), dtype=torch.float32, device=dev)
    call(
        "trnblas_hip_ozaki_hilo", slices, M, N, Kp, ptr(dA), dA.stride(1), dA.stride(0),
        ptr(dB), dB.stride(1), dB.stride(0), ptr(hilo), N, stream_of(dev),
    )  # fmt: skip
    return hilo


def triangle_nonzero(C: torch.Tensor, uplo: str) -> tuple[bool, bool]:
    """(uplo triangle has a nonzero, the other triangle has one) for a device
    n x n C (strict triangles; one pass, one 8-byte device-to-host read)."""
    dev = _require_device(C)
    code = _lib.DTYPE_CODES.get(C.dtype)
    if code is None or C.stride(1) != 1:
        up = bool(torch.triu(C, diagonal=1).ne(0).any())
        lo = bool(torch.tril(C, diagonal=-1).ne(0).any())
    else:
        flags = torch.empty(2, dtype=torch.int32, device=dev)
        n = C.shape[0]
        call(
            "trnblas_hip_triangle_nonzero", code, n, ptr(C), max(C.stride(0), n), ptr(flags),
            stream_of(dev),
        )  # fmt: skip
        up, lo = (bool(v) for v in flags.tolist())
    return (up, lo) if uplo == "upper" else (lo, up)
