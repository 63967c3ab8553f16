"""Oracle: the density-fitting metric stage of trnblas, restated.

Test infrastructure only (see oracle/__init__.py).

* `trsm_ref`            op(A) X = alpha B (side "left") or X op(A) = alpha B
                        (side "right") on the `uplo` triangle of A, diag
                        "unit" replacing its diagonal by ones — the reference's
                        torch body (trnblas/nki/dispatch.py:1707-1738, public
                        wrapper trnblas/level3.py:332-362) — in float64 numpy,
                        solved by a dense LU solve of the explicit triangular
                        matrix (no triangular solver involved);
* `metric_inv_half_ref` X = L^-T for J = L L^T (dispatch.py:1854-1881,
                        level3.py:365-380) as numpy.linalg.inv(L).T in
                        float64 from numpy's Cholesky;
* `spd`                 a seeded SPD matrix (the reference's test recipe,
                        tests/test_conformance.py:1010-1018, is S S^T + n I).

Pinned by tests/test_oracle_metric.py: trsm_ref with A = I returns alpha B,
with a diagonal A divides the rows (left) / columns (right) of B, a unit
diagonal ignores A's stored diagonal, the other triangle of A is never read
(filling it with NaN changes nothing), and the residual op(T) X - alpha B
vanishes for every flag combination; metric_inv_half_ref gives diag(d^-1/2)
for a diagonal J, the 2 x 2 closed form, an upper-triangular X with
X X^T J = I, and X^T J X = I.
"""

from __future__ import annotations

import numpy as np


def _tri(A: np.ndarray, uplo: str, diag: str) -> np.ndarray:
    T = np.triu(A) if uplo == "upper" else np.tril(A)
    if diag == "unit":
        # the diagonal is not read (BLAS); the reference's torch body writes
        # T - diag(diag(T)) + I, the same unless the stored diagonal is not finite
        np.fill_diagonal(T, 1.0)
    return T


def trsm_ref(alpha, A, B, side="left", uplo="upper", trans=False, diag="nonunit") -> np.ndarray:
    """Float64 X of the reference's trsm (dispatch.py:1707-1738)."""
    A = np.asarray(A, dtype=np.float64)
    B = np.asarray(B, dtype=np.float64)
    T = _tri(A, uplo, diag)
    M = T.T if trans else T
    if side == "left":  # M X = alpha B
        return np.linalg.solve(M, alpha * B) if B.size else np.zeros_like(B)
    # X M = alpha B  <=>  M^T X^T = alpha B^T
    return np.linalg.solve(M.T, alpha * B.T).T if B.size else np.zeros_like(B)


def metric_inv_half_ref(J) -> np.ndarray:
    """Float64 L^-T for J = L L^T (dispatch.py:1854-1881)."""
    J = np.asarray(J, dtype=np.float64)
    if J.shape[0] == 0:
        return np.zeros((0, 0))
    L = np.linalg.cholesky(J)
    return np.linalg.inv(L).T


def spd(n: int, seed: int = 0) -> np.ndarray:
    """A seeded, well-conditioned SPD matrix S S^T + n I (float64)."""
    rng = np.random.default_rng(seed)
    S = rng.standard_normal((n, n))
    return S @ S.T + n * np.eye(n)
