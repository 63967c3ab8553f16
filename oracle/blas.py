"""Oracle: Level-3 GEMM / batched GEMM / SYRK semantics of trnblas.

Test infrastructure only (see oracle/__init__.py).

Two forms of each op:
* `*_cpu`: the reference's CPU torch path (what `trnblas.gemm` etc. compute
  with no accelerator: `torch.matmul` in the operands' dtype, then the
  `_scale_add` epilogue, trnblas/level3.py:42-66, :69-134, :243-329);
* `*_f64`: the same closed form in float64 (the parity judge; the north
  star's fp32 GEMM gate is componentwise 1e-6 (|A||B|)ij).

Pinned by tests/test_oracle_blas.py: integer-valued operands whose products
are exact in fp32 and fp64 (cpu == f64 exactly), known answers for the
SYRK triangle rules (level3.py:263-270, :298-329; the reference's
test_conformance.py:819-905 cases), alpha / beta / transpose special cases
(alpha = 0, beta = 0 ignoring NaN in C, identity operands), and C never
mutated.
"""

from __future__ import annotations

import warnings

import torch


def _op(X: torch.Tensor, trans: bool) -> torch.Tensor:
    return X.mT if trans and X.dim() >= 2 else X


def scale_add(result: torch.Tensor, alpha: float, beta: float, C) -> torch.Tensor:
    """alpha * result + beta * C for a fresh `result` (level3.py:42-66); C is
    ignored when None or beta == 0, and never written."""
    out = result * alpha if alpha != 1.0 else result.clone()
    if C is not None and beta != 0.0:
        out = out + beta * C
    return out


def gemm_cpu(alpha, A, B, beta=0.0, C=None, transA=False, transB=False) -> torch.Tensor:
    """level3.py:69-109 on host tensors (the pytorch backend)."""
    return scale_add(torch.matmul(_op(A, transA), _op(B, transB)), alpha, beta, C)


def gemm_f64(alpha, A, B, beta=0.0, C=None, transA=False, transB=False) -> torch.Tensor:
    a, b = _op(A, transA).double().cpu(), _op(B, transB).double().cpu()
    R = alpha * torch.matmul(a, b)
    if C is not None and beta != 0.0:
        R = R + beta * C.double().cpu()
    return R


def gemm_cw_den(alpha, A, B, beta=0.0, C=None, transA=False, transB=False) -> torch.Tensor:
    """|alpha| (|op(A)| |op(B)|) + |beta| |C|: the componentwise scale of the
    GEMM error gate."""
    a, b = _op(A, transA).double().cpu().abs(), _op(B, transB).double().cpu().abs()
    den = abs(alpha) * torch.matmul(a, b)
    if C is not None and beta != 0.0:
        den = den + abs(beta) * C.double().cpu().abs()
    return den


def max_cw_err(D, den, ref) -> float:
    den = torch.where(den > 0, den, torch.ones_like(den))
    return float(((D.double().cpu() - ref) / den).abs().max())


def batched_gemm_cpu(alpha, A, B, beta=0.0, C=None, transA=False, transB=False):
    """level3.py:112-134: torch.matmul broadcasting over the batch dims."""
    a = A.transpose(-2, -1) if transA else A
    b = B.transpose(-2, -1) if transB else B
    return scale_add(torch.matmul(a, b), alpha, beta, C)


def sym_from_triangle(C: torch.Tensor, uplo: str) -> torch.Tensor:
    """level3.py:298-302: the symmetric matrix stored in `uplo` of C."""
    if uplo == "upper":
        return torch.triu(C) + torch.triu(C, diagonal=1).mT
    return torch.tril(C) + torch.tril(C, diagonal=-1).mT


def resolve_syrk_uplo(C: torch.Tensor, uplo: str) -> str:
    """level3.py:305-329: `uplo`, or the other triangle when only it holds
    off-diagonal entries (DeprecationWarning)."""
    has_upper = bool(torch.triu(C, diagonal=1).ne(0).any())
    has_lower = bool(torch.tril(C, diagonal=-1).ne(0).any())
    other = "lower" if uplo == "upper" else "upper"
    mine, theirs = (has_upper, has_lower) if uplo == "upper" else (has_lower, has_upper)
    if theirs and not mine:
        warnings.warn(f"syrk: using the {other} triangle of C", DeprecationWarning, stacklevel=2)
        return other
    return uplo


def symmetrize(S: torch.Tensor) -> torch.Tensor:
    """dispatch.py:3178-3199 values: 0.5 (S + S^T)."""
    return 0.5 * (S + S.mT)


def syrk_cpu(alpha, A, beta=0.0, C=None, trans=False, uplo="upper") -> torch.Tensor:
    """level3.py:243-295 on host tensors: full symmetric result."""
    Ae = A.mT if trans else A
    n = Ae.shape[0]
    S = torch.matmul(Ae, Ae.mT)
    add = C is not None and beta != 0.0
    if add and C.dim() == 2 and tuple(C.shape) == (n, n):
        Cs = sym_from_triangle(C, resolve_syrk_uplo(C, uplo))
        return scale_add(symmetrize(S), alpha, beta, Cs)
    if not add:
        return scale_add(symmetrize(S), alpha, beta, C)
    return symmetrize(scale_add(S, alpha, beta, C))


def syrk_f64(alpha, A, beta=0.0, C=None, trans=False, uplo="upper") -> torch.Tensor:
    Ae = (A.mT if trans else A).double().cpu()
    R = alpha * (Ae @ Ae.mT)
    if C is not None and beta != 0.0:
        Cd = C.double().cpu()
        R = R + beta * sym_from_triangle(Cd, resolve_syrk_uplo(Cd, uplo))
    return R
