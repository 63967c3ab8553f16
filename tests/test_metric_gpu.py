"""trsm / metric_inv_half on the MI355X (device-resident operands solve on
the device in their own precision, float64 included) against
oracle/metric.py. Gates: the residual max|J X X^T - I| (< 1e-10 in float64,
< 1e-3 in float32; tests/test_conformance.py:1010-1018) and componentwise
agreement with the float64 oracle."""

import itertools

import numpy as np
import pytest
import torch

import trnblas_amd as tb
from oracle import metric as om

pytestmark = pytest.mark.gpu

FLAGS = list(itertools.product(["left", "right"], ["upper", "lower"], [False, True], ["nonunit", "unit"]))


@pytest.mark.parametrize("side,uplo,trans,diag", FLAGS)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_trsm_device_flags(dev, side, uplo, trans, diag, dtype):
    g = torch.Generator().manual_seed(7)
    n, m = 129, 33
    # off-diagonal entries ~ 1/n keep the triangle well conditioned also for
    # diag="unit" (N(0, 1) entries under a unit diagonal grow the solution
    # exponentially in n)
    A = torch.randn(n, n, generator=g, dtype=torch.float64) / n + 2 * torch.eye(n, dtype=torch.float64)
    B = torch.randn((n, m) if side == "left" else (m, n), generator=g, dtype=torch.float64)
    X = tb.trsm(1.25, A.to(dev, dtype), B.to(dev, dtype), side=side, uplo=uplo, trans=trans, diag=diag)
    assert X.device.type == "cuda" and X.dtype == dtype and X.shape == B.shape
    want = om.trsm_ref(1.25, A.numpy(), B.numpy(), side, uplo, trans, diag)
    tol = 1e-12 if dtype == torch.float64 else 1e-4
    assert np.abs(X.double().cpu().numpy() - want).max() <= tol * np.abs(want).max()


def test_trsm_device_bf16_and_views(dev):
    g = torch.Generator().manual_seed(8)
    A = torch.randn(64, 64, generator=g, dtype=torch.float64) / 64 + 2 * torch.eye(64, dtype=torch.float64)
    B = torch.randn(64, 16, generator=g, dtype=torch.float64)
    want = om.trsm_ref(1.0, A.numpy(), B.numpy(), "left", "lower", True, "nonunit")
    Ad = A.to(dev).mT.contiguous().mT  # transposed storage
    X = tb.trsm(1.0, Ad, B.to(dev), uplo="lower", trans=True)
    assert np.abs(X.cpu().numpy() - want).max() < 1e-12 * np.abs(want).max()
    Xb = tb.trsm(1.0, A.to(dev, torch.bfloat16), B.to(dev, torch.bfloat16), uplo="lower", trans=True)
    assert Xb.dtype == torch.bfloat16
    assert np.abs(Xb.double().cpu().numpy() - want).max() < 3e-2 * np.abs(want).max()


@pytest.mark.parametrize("n", [1, 2, 127, 129, 1024])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_metric_inv_half_device(dev, n, dtype):
    J = torch.from_numpy(om.spd(n, seed=60 + n))
    X = tb.metric_inv_half(J.to(dev, dtype))
    assert X.device.type == "cuda" and X.dtype == dtype
    assert torch.equal(X, torch.triu(X))
    Xd, Jd = X.double(), J.to(dev)
    err = float((Jd @ Xd @ Xd.mT - torch.eye(n, dtype=torch.float64, device=dev)).abs().max())
    assert err < (1e-3 if dtype == torch.float32 else 1e-10)
    want = om.metric_inv_half_ref(J.numpy())
    tol = 1e-12 if dtype == torch.float64 else 1e-4
    assert np.abs(Xd.cpu().numpy() - want).max() <= tol * np.abs(want).max()


def test_metric_inv_half_device_naux4096_fp64(dev):
    # the DF metric size of configs 3/4 (naux <= 4096): float64 on the device
    n = 4096
    g = torch.Generator(device=dev).manual_seed(11)
    S = torch.randn(n, n, generator=g, dtype=torch.float64, device=dev)
    J = S @ S.mT / n + torch.eye(n, dtype=torch.float64, device=dev)
    X = tb.metric_inv_half(J)
    assert torch.equal(X, torch.triu(X))
    err = float((J @ X @ X.mT - torch.eye(n, dtype=torch.float64, device=dev)).abs().max())
    assert err < 1e-10, err


def test_metric_inv_half_device_errors(dev):
    with pytest.raises(torch.linalg.LinAlgError):
        tb.metric_inv_half(-torch.eye(5, dtype=torch.float64, device=dev))
    with pytest.raises(NotImplementedError):
        tb.metric_inv_half(torch.eye(3, dtype=torch.int32, device=dev))
    assert tb.metric_inv_half(torch.zeros(0, 0, device=dev)).shape == (0, 0)


@pytest.mark.parametrize("nb", [1, 5, 64, 127, 128])
def test_chol_block_kernel(dev, nb):
    # one diagonal block through the C ABI: L L^T = A, L L^-1 = I, L^-1 equal
    # to the oracle's inverse Cholesky factor; the strict upper triangle of
    # A is neither read nor written
    from trnblas_amd.hip import kernels

    J = om.spd(nb, seed=nb)
    A = torch.from_numpy(J).to(dev)
    A_up = torch.triu(torch.full((nb, nb), 7.0, dtype=torch.float64, device=dev), 1)
    A = torch.tril(A) + A_up
    Li = torch.empty(nb, nb, dtype=torch.float64, device=dev)
    info = torch.zeros(1, dtype=torch.int32, device=dev)
    kernels.chol_block(A, Li, info, 0)
    assert int(info) == 0
    assert torch.equal(torch.triu(A, 1), A_up)
    L = torch.tril(A).cpu().numpy()
    assert np.abs(L @ L.T - J).max() <= 1e-13 * np.abs(J).max()
    Lin = Li.cpu().numpy()
    assert np.array_equal(Lin, np.tril(Lin))
    assert np.abs(L @ Lin - np.eye(nb)).max() <= 1e-13
    want = om.metric_inv_half_ref(J).T  # L^-1
    assert np.abs(Lin - want).max() <= 1e-12 * np.abs(want).max()


def test_chol_block_info(dev):
    # the first non-positive pivot, offset by the block's position, and an
    # info already set by an earlier block is kept
    from trnblas_amd.hip import kernels

    A = torch.eye(10, dtype=torch.float64, device=dev)
    A[6, 6] = -1.0
    Li = torch.empty_like(A)
    info = torch.zeros(1, dtype=torch.int32, device=dev)
    kernels.chol_block(A.clone(), Li, info, 100)
    assert int(info) == 107
    kernels.chol_block(A.clone(), Li, info, 500)
    assert int(info) == 107
    info.zero_()
    A[6, 6] = float("nan")
    kernels.chol_block(A.clone(), Li, info, 0)
    assert int(info) == 7


@pytest.mark.parametrize("n", [300, 385])
@pytest.mark.parametrize("cond", [1e2, 1e8])
def test_metric_inv_half_blocked_conditioning(dev, n, cond):
    # several 128-wide blocks, a ragged last one, and RI-like conditioning:
    # the residual stays within a small factor of LAPACK's on the same J
    rng = np.random.default_rng(int(n + np.log10(cond)))
    Q, _ = np.linalg.qr(rng.standard_normal((n, n)))
    J = (Q * np.geomspace(1.0, 1.0 / cond, n)) @ Q.T
    J = (J + J.T) / 2
    X = tb.metric_inv_half(torch.from_numpy(J).to(dev)).cpu().numpy()
    assert np.array_equal(X, np.triu(X))
    res = np.abs(X.T @ J @ X - np.eye(n)).max()
    Xh = om.metric_inv_half_ref(J)
    res_h = np.abs(Xh.T @ J @ Xh - np.eye(n)).max()
    assert res <= 20 * res_h + 1e-13, (res, res_h)
    assert np.abs(X - Xh).max() <= 1e-14 * cond * np.abs(Xh).max()


def test_metric_inv_half_device_error_later_block(dev):
    # a failing leading minor inside the third block is reported by its order
    J = torch.eye(300, dtype=torch.float64, device=dev)
    J[261, 261] = -2.0
    with pytest.raises(torch.linalg.LinAlgError, match="order 262"):
        tb.metric_inv_half(J)


def _trsm_case(n, m, side, seed):
    g = torch.Generator().manual_seed(seed)
    A = torch.randn(n, n, generator=g, dtype=torch.float64) / n + 2 * torch.eye(n, dtype=torch.float64)
    B = torch.randn((n, m) if side == "left" else (m, n), generator=g, dtype=torch.float64)
    return A, B


@pytest.mark.parametrize("n,m", [(300, 70), (1000, 700)])
@pytest.mark.parametrize("side,uplo,trans,diag", FLAGS)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_trsm_device_flags_multiblock(dev, n, m, side, uplo, trans, diag, dtype):
    """3 and 8 diagonal blocks of 128 (uneven halving, nested updates), ragged
    n, nrhs above one GEMM tile, right solves through strided views."""
    A, B = _trsm_case(n, m, side, 100 + n)
    X = tb.trsm(0.75, A.to(dev, dtype), B.to(dev, dtype), side=side, uplo=uplo, trans=trans, diag=diag)
    assert X.device.type == "cuda" and X.dtype == dtype and X.shape == B.shape
    want = om.trsm_ref(0.75, A.numpy(), B.numpy(), side, uplo, trans, diag)
    tol = 1e-12 if dtype == torch.float64 else 1e-4
    assert np.abs(X.double().cpu().numpy() - want).max() <= tol * np.abs(want).max()


@pytest.mark.parametrize("side,uplo,trans,diag", [("left", "lower", False, "nonunit"),
                                                  ("right", "upper", True, "unit"),
                                                  ("left", "upper", True, "nonunit"),
                                                  ("right", "lower", False, "nonunit")])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_trsm_device_large(dev, side, uplo, trans, diag, dtype):
    n, m = 2500, 600  # 20 blocks, the last ragged
    A, B = _trsm_case(n, m, side, 7)
    X = tb.trsm(1.0, A.to(dev, dtype), B.to(dev, dtype), side=side, uplo=uplo, trans=trans, diag=diag)
    want = om.trsm_ref(1.0, A.numpy(), B.numpy(), side, uplo, trans, diag)
    tol = 1e-12 if dtype == torch.float64 else 1e-4
    assert np.abs(X.double().cpu().numpy() - want).max() <= tol * np.abs(want).max()


@pytest.mark.parametrize("side", ["left", "right"])
def test_trsm_device_ill_conditioned(dev, side):
    """A Cholesky factor with cond ~1e4 (an SPD matrix of eigenvalues 1 .. 1e-8):
    the block inverses of the diagonal are where such a triangle loses
    accuracy. fp64 against torch's solve_triangular on the same device, with
    a backward-error (residual) gate and a forward gate scaled by cond."""
    n, m = 1000, 300
    rng = np.random.default_rng(5)
    Q, _ = np.linalg.qr(rng.standard_normal((n, n)))
    J = (Q * np.logspace(0, -8, n)) @ Q.T
    L = np.linalg.cholesky((J + J.T) / 2)
    B = rng.standard_normal((n, m) if side == "left" else (m, n))
    Ld, Bd = torch.from_numpy(L).to(dev), torch.from_numpy(B).to(dev)
    X = tb.trsm(1.0, Ld, Bd, side=side, uplo="lower")
    if side == "left":
        ref = torch.linalg.solve_triangular(Ld, Bd, upper=False)
        res = Ld @ X - Bd
    else:
        ref = torch.linalg.solve_triangular(Ld, Bd, upper=False, left=False)
        res = X @ Ld - Bd
    scale = float(Ld.abs().max()) * float(X.abs().max()) * n
    assert float(res.abs().max()) <= 1e-13 * scale
    cond = np.linalg.cond(L)
    assert float((X - ref).abs().max()) <= 1e-14 * cond * float(ref.abs().max())


def test_metric_solve_host_route(dev, monkeypatch):
    # TRNBLAS_METRIC_SOLVE=host (nki/dispatch.py:1833-1870): host LAPACK in
    # fp64, the factor back on J's device in J's dtype
    J = torch.from_numpy(om.spd(300, seed=9))
    monkeypatch.setenv("TRNBLAS_METRIC_SOLVE", "host")
    X = tb.metric_inv_half(J.to(dev, torch.float32))
    assert X.device.type == "cuda" and X.dtype == torch.float32
    want = om.metric_inv_half_ref(J.numpy())
    assert np.abs(X.double().cpu().numpy() - want).max() <= 1e-6 * np.abs(want).max()
    monkeypatch.setenv("TRNBLAS_METRIC_SOLVE", "device")
    Xd = tb.metric_inv_half(J.to(dev))
    assert np.abs(Xd.cpu().numpy() - want).max() <= 1e-12 * np.abs(want).max()
