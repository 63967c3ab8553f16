"""trsm / metric_inv_half on host tensors (the host route of the product,
CPU-only) against oracle/metric.py, with the reference's flag, dtype,
layout, empty-shape and error semantics (tests/test_conformance.py:985-1024,
tests/test_native_dispatch.py:812-910)."""

import itertools

import numpy as np
import pytest
import torch

import trnblas_amd as tb
from oracle import metric as om

FLAGS = list(itertools.product(["left", "right", "L", "r"], ["upper", "lower", "U", "l"], [False, True, "N", "T"], ["nonunit", "unit"]))
SIDE = {"left": "left", "L": "left", "right": "right", "r": "right"}
UPLO = {"upper": "upper", "U": "upper", "lower": "lower", "l": "lower"}


def _case(side, n=9, m=4, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    A = torch.randn(n, n, generator=g, dtype=torch.float64) + 4 * torch.eye(n, dtype=torch.float64)
    B = torch.randn((n, m) if side == "left" else (m, n), generator=g, dtype=torch.float64)
    return A.to(dtype), B.to(dtype)


@pytest.mark.parametrize("side,uplo,trans,diag", FLAGS[::3])
def test_trsm_host_flags(side, uplo, trans, diag):
    s, u = SIDE[side], UPLO[uplo]
    t = trans in (True, "T")
    A, B = _case(s, seed=len(side) + len(uplo))
    X = tb.trsm(0.75, A, B, side=side, uplo=uplo, trans=trans, diag=diag)
    want = om.trsm_ref(0.75, A.numpy(), B.numpy(), s, u, t, diag)
    assert X.dtype == torch.float64 and X.shape == B.shape
    assert np.abs(X.numpy() - want).max() <= 1e-12 * max(1.0, np.abs(want).max())


def test_trsm_host_layouts_dtypes_and_empty():
    A, B = _case("left", n=65, m=33, seed=3)
    want = om.trsm_ref(1.0, A.numpy(), B.numpy(), "left", "lower", False, "nonunit")
    At = A.mT.contiguous().mT  # transposed storage, same values
    X = tb.trsm(1.0, At, B[:, :], uplo="lower")
    assert np.abs(X.numpy() - want).max() < 1e-11
    X32 = tb.trsm(1.0, A.float(), B.float(), uplo="lower")
    assert X32.dtype == torch.float32
    assert np.abs(X32.double().numpy() - want).max() < 1e-4 * np.abs(want).max()
    Xb = tb.trsm(1.0, A.bfloat16(), B.bfloat16(), uplo="lower")  # solved in fp32
    assert Xb.dtype == torch.bfloat16
    Xe = tb.trsm(1.0, torch.eye(0, dtype=torch.float64), torch.zeros(0, 3, dtype=torch.float64))
    assert Xe.shape == (0, 3)


def test_trsm_host_errors():
    A, B = _case("left")
    with pytest.raises(ValueError):
        tb.trsm(1.0, A, B, side="middle")
    with pytest.raises(ValueError):
        tb.trsm(1.0, A, B, uplo="diagonal")
    with pytest.raises(ValueError):
        tb.trsm(1.0, A, B, trans="C")
    with pytest.raises(ValueError):
        tb.trsm(1.0, A, B, diag="x")
    with pytest.raises(ValueError):
        tb.trsm(1.0, A, B.mT)  # B rows must match A for side="left"


def test_trsm_host_keeps_autograd():
    A, B = _case("left", n=6, m=2, seed=5)
    A.requires_grad_(True)
    B.requires_grad_(True)
    tb.trsm(1.0, A, B, uplo="lower").sum().backward()
    assert A.grad is not None and B.grad is not None
    assert torch.equal(A.grad.triu(1), torch.zeros_like(A.grad).triu(1))  # upper never read


@pytest.mark.parametrize("n", [1, 2, 127, 129])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_metric_inv_half_host(n, dtype):
    J = torch.from_numpy(om.spd(n, seed=60 + n)).to(dtype)
    X = tb.metric_inv_half(J)
    assert X.dtype == dtype and torch.equal(X, torch.triu(X))
    Xd = X.double()
    err = float((J.double() @ Xd @ Xd.mT - torch.eye(n, dtype=torch.float64)).abs().max())
    assert err < (1e-3 if dtype == torch.float32 else 1e-10)
    want = om.metric_inv_half_ref(J.double().numpy())
    assert np.abs(Xd.numpy() - want).max() <= (1e-4 if dtype == torch.float32 else 1e-12) * np.abs(want).max()


def test_metric_inv_half_host_errors_and_empty():
    assert tb.metric_inv_half(torch.zeros(0, 0)).shape == (0, 0)
    with pytest.raises(NotImplementedError):
        tb.metric_inv_half(torch.eye(3, dtype=torch.int64))
    with pytest.raises(torch.linalg.LinAlgError):
        tb.metric_inv_half(-torch.eye(3, dtype=torch.float64))
    Jt = torch.from_numpy(om.spd(40, seed=2)).mT  # transposed layout
    X = tb.metric_inv_half(Jt)
    assert float((Jt @ X @ X.mT - torch.eye(40, dtype=torch.float64)).abs().max()) < 1e-10
