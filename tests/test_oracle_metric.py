"""Pins oracle/metric.py (CPU): closed forms and invariants that a dropped
term, a wrong triangle, a missed transpose or a wrong side would fail."""

import itertools

import numpy as np
import pytest

from oracle import metric as om

FLAGS = list(itertools.product(["left", "right"], ["upper", "lower"], [False, True], ["nonunit", "unit"]))


def _op_tri(A, uplo, trans, diag):
    T = np.triu(A) if uplo == "upper" else np.tril(A)
    if diag == "unit":
        np.fill_diagonal(T, 1.0)
    return T.T if trans else T


@pytest.mark.parametrize("side,uplo,trans,diag", FLAGS)
def test_trsm_ref_residual_and_unread_triangle(side, uplo, trans, diag):
    rng = np.random.default_rng(hash((side, uplo, trans, diag)) % 1000)
    n = 7
    A = rng.standard_normal((n, n)) + 4 * np.eye(n)
    B = rng.standard_normal((n, 3) if side == "left" else (3, n))
    X = om.trsm_ref(1.5, A, B, side, uplo, trans, diag)
    M = _op_tri(A, uplo, trans, diag)
    R = M @ X if side == "left" else X @ M
    assert np.abs(R - 1.5 * B).max() < 1e-12
    # the other triangle (and, for a unit diagonal, the diagonal) is never read
    A2 = A.copy()
    other = np.tril_indices(n, -1) if uplo == "upper" else np.triu_indices(n, 1)
    A2[other] = np.nan
    if diag == "unit":
        np.fill_diagonal(A2, np.nan)
    assert np.array_equal(om.trsm_ref(1.5, A2, B, side, uplo, trans, diag), X)


def test_trsm_ref_closed_forms():
    rng = np.random.default_rng(1)
    B = rng.standard_normal((4, 5))
    assert np.allclose(om.trsm_ref(2.0, np.eye(4), B), 2.0 * B, rtol=0, atol=1e-15)
    d = np.array([2.0, -4.0, 0.5, 8.0])
    assert np.allclose(om.trsm_ref(1.0, np.diag(d), B, side="left"), B / d[:, None], rtol=1e-15)
    Bt = B.T
    assert np.allclose(om.trsm_ref(1.0, np.diag(d), Bt, side="right"), Bt / d[None, :], rtol=1e-15)
    # upper 2 x 2 by back substitution: [[a, b], [0, c]] x = y
    a, b, c = 2.0, 3.0, 4.0
    y = np.array([[5.0], [8.0]])
    x1 = 8.0 / c
    x0 = (5.0 - b * x1) / a
    assert np.allclose(om.trsm_ref(1.0, [[a, b], [9.0, c]], y), [[x0], [x1]], rtol=1e-15)
    # ... and transposed: [[a, 0], [b, c]] x = y by forward substitution
    z0 = 5.0 / a
    z1 = (8.0 - b * z0) / c
    assert np.allclose(om.trsm_ref(1.0, [[a, b], [9.0, c]], y, trans=True), [[z0], [z1]], rtol=1e-15)


def test_metric_inv_half_ref_closed_forms():
    d = np.array([4.0, 9.0, 0.25])
    X = om.metric_inv_half_ref(np.diag(d))
    assert np.allclose(X, np.diag(1.0 / np.sqrt(d)), rtol=1e-15)
    # 2 x 2: J = [[p, q], [q, r]], L = [[sqrt p, 0], [q / sqrt p, s]], s^2 = r - q^2 / p
    p, q, r = 4.0, 2.0, 5.0
    lp, s = np.sqrt(p), np.sqrt(r - q * q / p)
    L = np.array([[lp, 0.0], [q / lp, s]])
    want = np.linalg.inv(L).T
    assert np.allclose(want, [[1 / lp, -q / (lp * lp * s)], [0.0, 1 / s]], rtol=1e-15)
    assert np.allclose(om.metric_inv_half_ref([[p, q], [q, r]]), want, rtol=1e-15)
    assert om.metric_inv_half_ref(np.zeros((0, 0))).shape == (0, 0)


@pytest.mark.parametrize("n", [1, 2, 31, 130])
def test_metric_inv_half_ref_defining_property(n):
    J = om.spd(n, seed=n)
    X = om.metric_inv_half_ref(J)
    assert np.array_equal(X, np.triu(X))
    assert np.abs(J @ X @ X.T - np.eye(n)).max() < 1e-12
    assert np.abs(X.T @ J @ X - np.eye(n)).max() < 1e-12
