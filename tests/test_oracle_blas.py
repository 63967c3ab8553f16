"""Pins of the Level-3 oracle (oracle/blas.py), CPU only."""

import warnings

import pytest
import torch

from oracle import blas


def _ints(*shape, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-8, 9, shape, generator=g).float()


def test_gemm_cpu_exact_on_integers():
    A, B, C = _ints(7, 11, seed=1), _ints(11, 5, seed=2), _ints(7, 5, seed=3)
    for ta, tb in [(False, False), (True, False), (False, True), (True, True)]:
        a = A.mT.contiguous() if ta else A
        b = B.mT.contiguous() if tb else B
        got = blas.gemm_cpu(2.0, a, b, 0.5, C, transA=ta, transB=tb)
        assert torch.equal(got.double(), blas.gemm_f64(2.0, a, b, 0.5, C, transA=ta, transB=tb))
        assert torch.equal(got, 2.0 * (A @ B) + 0.5 * C)


def test_gemm_beta_zero_ignores_nan_c_and_never_writes_c():
    A, B = _ints(4, 3), _ints(3, 2, seed=4)
    C = torch.full((4, 2), float("nan"))
    before = C.clone()
    out = blas.gemm_cpu(1.0, A, B, 0.0, C)
    assert torch.isfinite(out).all()
    assert torch.equal(C.isnan(), before.isnan())


def test_gemm_alpha_zero_and_identity():
    A = _ints(5, 5)
    assert torch.equal(blas.gemm_cpu(0.0, A, A), torch.zeros(5, 5))
    assert torch.equal(blas.gemm_cpu(1.0, A, torch.eye(5)), A)


def test_syrk_triangle_rules():
    A = _ints(6, 4, seed=5)
    X = _ints(6, 6, seed=6)
    lower = torch.tril(X) + torch.tril(X, -1).T
    for uplo in ("lower", "upper"):
        out = blas.syrk_cpu(1.0, A, 0.5, X, uplo=uplo)
        Cs = lower if uplo == "lower" else torch.triu(X) + torch.triu(X, 1).T
        assert torch.equal(out, A @ A.T + 0.5 * Cs)
        assert torch.equal(out, out.T)
    # only the other triangle stored: used, with a DeprecationWarning
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        out = blas.syrk_cpu(1.0, A, 0.5, torch.tril(X), uplo="upper")
    assert any(issubclass(x.category, DeprecationWarning) for x in w)
    assert torch.equal(out, A @ A.T + 0.5 * lower)


def test_syrk_trans_and_broadcast_c():
    A = _ints(4, 6, seed=7)
    out = blas.syrk_cpu(1.0, A, trans=True)
    assert torch.equal(out, A.T @ A)
    out = blas.syrk_cpu(2.0, A, 1.0, torch.tensor(3.0))
    assert torch.equal(out, 2.0 * (A @ A.T) + 3.0)


@pytest.mark.parametrize("shape", [(3, 4, 5), (1, 2, 2)])
def test_batched_gemm_broadcast(shape):
    b, m, k = shape
    A = _ints(b, m, k, seed=8)
    B = _ints(k, 3, seed=9)
    assert torch.equal(blas.batched_gemm_cpu(1.0, A, B), A @ B)
