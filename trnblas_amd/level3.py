"""BLAS Level 3 on MI355X: gemm, batched_gemm, syrk, gemm_fp64, and the
density-fitting metric stage trsm / metric_inv_half.

Same signatures, flags and result semantics as trnblas/level3.py (drop-in):
* `gemm` / `batched_gemm` (level3.py:69-134): C = alpha op(A) op(B) + beta C
  into a fresh tensor, C never written, torch.matmul broadcasting;
* `syrk` (level3.py:243-329): the full symmetric result, only the `uplo`
  triangle of an n x n C referenced (the other-triangle fallback with a
  DeprecationWarning kept);
* `gemm_fp64` (level3.py:137-193): fp64-class product by Ozaki splitting,
  `slices` in [1, 12], float64 result on A's device;
* `trsm` / `metric_inv_half` (level3.py:332-380): triangular solve and the
  Cholesky inverse factor L^-T, on the operands' device in their precision
  (float64 native on the MI355X).

On a ROCm GPU the operands run the gfx950 kernels of `libtrnblas_hip.so`
with transposes read in place and the alpha / beta epilogue fused into the
kernel's store; see `hip/dispatch.py` for the routing.
"""

from __future__ import annotations

import warnings

import torch

from ._flags import diag_flag, side_flag, trans_flag, uplo_flag
from .hip import dispatch as _d
from .hip._lib import broadcast_shapes as _broadcast_shapes


def _owned_inplace_ok(result: torch.Tensor) -> bool:
    return (
        not (torch.is_grad_enabled() and result.requires_grad)
        and result.is_contiguous()
        and (result.is_floating_point() or result.is_complex())
    )


def _scale_add(result: torch.Tensor, alpha: float, beta: float, C) -> torch.Tensor:
    """alpha * result + beta * C for a fresh `result` the wrapper owns,
    updated in place when that keeps its dtype / layout (level3.py:42-66)."""
    add = C is not None and beta != 0.0
    inplace = _owned_inplace_ok(result)
    if inplace and add:
        inplace = (
            C.dtype == result.dtype
            and C.device == result.device
            and _broadcast_shapes(result.shape, C.shape) == tuple(result.shape)
        )
    if not inplace:
        result = alpha * result
        return result + beta * C if add else result
    if alpha != 1.0:
        result.mul_(alpha)
    if add:
        result.add_(C, alpha=beta)
    return result


def gemm(
    alpha: float,
    A: torch.Tensor,
    B: torch.Tensor,
    beta: float = 0.0,
    C: torch.Tensor | None = None,
    transA: bool = False,
    transB: bool = False,
) -> torch.Tensor:
    """General matrix multiply: alpha * op(A) @ op(B) + beta * C.

    op(X) = X, or X with its last two dims transposed when trans. A
    transposed operand is read in place by the kernel (no copy).
    """
    D = _d.gemm_fast(alpha, A, B, beta, C, transA, transB)
    if D is not None:
        return D
    transA, transB = trans_flag(transA, "transA"), trans_flag(transB, "transB")
    a = A.mT if transA and A.dim() >= 2 else A
    b = B.mT if transB and B.dim() >= 2 else B
    if a.dim() >= 2 and b.dim() >= 2 and a.dim() <= 3 and b.dim() <= 3:
        return _d.gemm_scaled(alpha, a, b, beta, C)
    return _scale_add(torch.matmul(a, b), alpha, beta, C)


def batched_gemm(
    alpha: float,
    A: torch.Tensor,
    B: torch.Tensor,
    beta: float = 0.0,
    C: torch.Tensor | None = None,
    transA: bool = False,
    transB: bool = False,
) -> torch.Tensor:
    """Batched GEMM: C[i] = alpha * op(A[i]) @ op(B[i]) + beta * C[i] with
    torch.matmul batch broadcasting; one kernel launch for the whole batch."""
    transA, transB = trans_flag(transA, "transA"), trans_flag(transB, "transB")
    a = A.transpose(-2, -1) if transA else A
    b = B.transpose(-2, -1) if transB else B
    if a.dim() == 3 and b.dim() == 3:
        return _d.gemm_scaled(alpha, a, b, beta, C)
    return _scale_add(_d.nki_batched_gemm(a, b), alpha, beta, C)


def gemm_fp64(
    A: torch.Tensor,
    B: torch.Tensor,
    *,
    slices: int = 8,
    transA: bool = False,
    transB: bool = False,
    mode: str | None = None,
) -> torch.Tensor:
    """fp64-class op(A) @ op(B) by Ozaki splitting on int8 MFMA.

    A is split row by row and B column by column into `slices` (k) int8
    digits of 7 bits, exactly; the k (k + 1) / 2 slice products run as int8
    MFMAs, all on the device. mode "exact" sums exact int32 groups of at most
    4096 terms into an fp32 TwoSum (hi, lo) pair in the reference's order and
    recombines in fp64 with the power-of-two scales: the result equals the
    reference's `ozaki.reference_gemm` bit for bit. mode "fast" (the default,
    TRNBLAS_OZAKI_MODE) sums each diagonal of slice pairs exactly in int32 and
    recombines all diagonals in fp64: same digits, same products, an error
    within the same truncation bound, not bitwise. mode "crt" (Ozaki scheme
    II) rounds each operand to the precision of k digits as one integer
    (p = 7k - 1 bits below its row / column maximum) and forms the integer
    product exactly from one int8 GEMM per modulus of a Chinese-remainder
    basis: within the same bound (no digit products are dropped), in
    n_moduli(k, K) GEMMs (16 at k = 8, 22 at k = 11 for K = 8192) instead of
    k (k + 1) / 2 (36, 66). Accuracy (max |C - C_exact| / (|A| |B|), normal
    data): about 1e-12 at k = 6, 1e-14 at k = 7, 2e-16 to 3e-16 at k = 8
    (the default, host-fp64 level); scaling is per row of A and column of B,
    so data spread over 10^+-4 needs k = 10, and entries 2^round(N(0, 16))
    times N(0, 1) at 8192^3 need k = 11 in mode "fast" and k = 10 in mode
    "crt" to match a host fp64 product. 1 <= slices <= 12.

    A (M, K) and B (K, N) are 2-D real tensors of any float dtype (computed as
    fp64). Returns float64 (M, N) on A's device. Without a ROCm GPU, under
    set_backend("pytorch") and for non-finite operands the result is an fp64
    matmul.
    """
    from .ozaki import check_mode, check_slices

    slices = check_slices(slices)
    mode = check_mode(mode)
    transA, transB = trans_flag(transA, "transA"), trans_flag(transB, "transB")
    for name, X in (("A", A), ("B", B)):
        if not isinstance(X, torch.Tensor) or X.dim() != 2:
            raise ValueError(f"gemm_fp64: {name} must be a 2-D tensor")
        if not X.is_floating_point():
            raise TypeError(f"gemm_fp64: {name} must be a real floating tensor, got {X.dtype}")
    a = A.mT if transA else A
    b = B.mT if transB else B
    if a.shape[1] != b.shape[0]:
        raise ValueError(
            f"gemm_fp64: inner dimensions differ: op(A) {tuple(a.shape)}, op(B) {tuple(b.shape)}"
        )
    device = A.device
    return _d.nki_gemm_fp64(a.detach(), b.detach(), slices, mode).to(device)


def syrk(
    alpha: float,
    A: torch.Tensor,
    beta: float = 0.0,
    C: torch.Tensor | None = None,
    trans: bool = False,
    uplo: str = "upper",
) -> torch.Tensor:
    """Symmetric rank-k update, returned as the full symmetric matrix:
    alpha * A @ A^T + beta * C (trans=False) or alpha * A^T @ A + beta * C.

    As in BLAS, only the `uplo` triangle of an n x n C is referenced. A C whose
    off-diagonal entries are all in the opposite triangle uses that triangle,
    with a DeprecationWarning. A C that broadcasts against the result (scalar,
    row, column) is added and the sum symmetrised. The kernel computes the
    lower triangle of the product only (n (n + 1) k flops) and writes each
    value to both positions, so the result is exactly symmetric.
    """
    trans = trans_flag(trans)
    uplo = uplo_flag(uplo)
    n = A.shape[1] if trans else A.shape[0]
    add = C is not None and beta != 0.0
    if add and C.dim() == 2 and tuple(C.shape) == (n, n):
        if C.dtype == A.dtype:
            res = _d.hip_syrk_checked(alpha, A, beta, C, trans, uplo)
            if res is not None:
                out, mine, theirs = res
                _syrk_side(uplo, mine, theirs)
                return out
        side = _resolve_syrk_uplo(C, uplo)
        Cs = _sym_from_triangle(C, side)
        A_eff = A.mT if trans else A
        return _scale_add(_d.nki_syrk(A_eff, symmetrize=True), alpha, beta, Cs)
    if not add:
        out = _d.hip_syrk(alpha, A, 0.0, None, trans, "lower")
        if out is not None:
            return out
    A_eff = A.mT if trans else A
    result = _scale_add(_d.nki_syrk(A_eff, symmetrize=not add), alpha, beta, C)
    return _d._symmetrize(result) if add else result


def _sym_from_triangle(C: torch.Tensor, uplo: str) -> torch.Tensor:
    """The symmetric matrix stored in the `uplo` triangle of C."""
    if uplo == "upper":
        return torch.triu(C) + torch.triu(C, diagonal=1).mT
    return torch.tril(C) + torch.tril(C, diagonal=-1).mT


def _resolve_syrk_uplo(C: torch.Tensor, uplo: str) -> str:
    """`uplo`, or the opposite triangle when only that one holds off-diagonal
    entries (level3.py:305-329). Checks the `uplo` triangle first, so a
    C with entries there costs one pass."""
    from .hip import kernels

    if C.device.type == "cuda" and _d._use_hip():
        mine, theirs = kernels.triangle_nonzero(C, uplo)
    else:
        up = bool(torch.triu(C, diagonal=1).ne(0).any())
        lo = bool(torch.tril(C, diagonal=-1).ne(0).any())
        mine, theirs = (up, lo) if uplo == "upper" else (lo, up)
    return _syrk_side(uplo, mine, theirs, stacklevel=4)


def _syrk_side(uplo: str, mine: bool, theirs: bool, stacklevel: int = 3) -> str:
    """The triangle rule (level3.py:305-329): `uplo`, or the other triangle,
    with a DeprecationWarning, when only that one holds off-diagonal entries."""
    other = "lower" if uplo == "upper" else "upper"
    if theirs and not mine:
        warnings.warn(
            f"syrk: C stores its off-diagonal entries only in the {other} triangle "
            f"but uplo={uplo!r}; using the {other} triangle. Pass uplo={other!r}. "
            "Only the uplo triangle of C is referenced when both are stored, and "
            "this fallback will be removed.",
            DeprecationWarning,
            stacklevel=stacklevel,
        )
        return other
    return uplo


def trsm(
    alpha: float,
    A: torch.Tensor,
    B: torch.Tensor,
    side: str = "left",
    uplo: str = "upper",
    trans: bool = False,
    diag: str = "nonunit",
) -> torch.Tensor:
    """Triangular solve with multiple right-hand sides (level3.py:332-362):
    op(A) @ X = alpha * B (side="left") or X @ op(A) = alpha * B
    (side="right"), op(A) = A or A^T. Only the `uplo` triangle of A is
    referenced; diag="unit" takes its diagonal as ones. Returns X with B's
    dtype and device. For DF: J = L L^T, L X = (mu nu|P).

    Device operands solve on the device in their own precision (float64
    included); see `hip.dispatch.nki_trsm`.
    """
    side, uplo, diag = side_flag(side), uplo_flag(uplo), diag_flag(diag)
    trans = trans_flag(trans)
    return _d.nki_trsm(A, B, side=side, uplo=uplo, trans=trans, diag=diag, alpha=alpha)


def metric_inv_half(J: torch.Tensor) -> torch.Tensor:
    """Cholesky inverse factor of an SPD metric (level3.py:365-380):
    X = L^-T where J = L @ L^T, so X @ X^T = J^-1 and `(ia|Q) @ X` is the
    density-fitting contraction B_ia^P = sum_Q (ia|Q) [J^-1/2]_QP. X is upper
    triangular, with J's dtype and device; a J that is not positive definite
    raises torch.linalg.LinAlgError, an integer J NotImplementedError.
    """
    return _d.nki_metric_inv_half(J)
