"""GPU parity of the Ozaki kernels (C ABI via trnblas_amd.hip.kernels):
digits and exponents bit-equal to the oracle split, (hi, lo) and the fp64
product bit-equal to the oracle's `reference_gemm`."""

import numpy as np
import pytest
import torch

from oracle import ozaki as oz
from oracle.exact import inputs

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("per", ["row", "col"])
@pytest.mark.parametrize("k", [1, 3, 8, 12])
def test_split_equals_oracle(dev, per, k):
    from trnblas_amd.hip import kernels

    rng = np.random.default_rng(k)
    X = rng.standard_normal((150, 300)) * 10.0 ** rng.uniform(-30, 30, (150, 300))
    X[3] = 0.0
    X[:, 7] = 0.0
    X[5, 9] = 5e-324
    d, e, bad = kernels.ozaki_split(torch.from_numpy(X).to(dev), k, per)
    torch.cuda.synchronize()
    assert int(bad) == 0
    want_d, want_e = oz.split(X, k, per=per, pad=(128, 128))
    got_d = d.cpu().numpy()
    if per == "col":  # device layout is (k, C, R): K (= R) contiguous
        got_d = got_d.transpose(0, 2, 1)
    R, C = X.shape
    assert np.array_equal(e.cpu().numpy().astype(np.int64), want_e)
    assert np.array_equal(got_d[:, :R, :C], want_d[:, :R, :C])
    assert not got_d[:, R:, :].any() and not got_d[:, :, C:].any()


def test_split_two_factor_and_nonfinite(dev):
    from trnblas_amd.hip import kernels

    X = np.array([[1e-310, 2e-311, 0.0], [1e300, -3.0, 1.0], [1.5, 2.5, -7.0]])
    d, e, bad = kernels.ozaki_split(torch.from_numpy(X).to(dev), 8, "row")
    want_d, want_e = oz.split(X, 8, per="row", pad=(128, 128))
    assert int(bad) == 0
    assert np.array_equal(e.cpu().numpy(), want_e)
    assert np.array_equal(d.cpu().numpy()[:, :3, :3], want_d[:, :3, :3])
    Y = X.copy()
    Y[1, 1] = np.inf
    _, _, bad = kernels.ozaki_split(torch.from_numpy(Y).to(dev), 8, "row")
    assert int(bad) == 1


@pytest.mark.parametrize(
    "M,K,N,k", [(64, 64, 64, 8), (37, 300, 53, 7), (130, 4100, 7, 8), (200, 9000, 31, 8),
                (1, 1, 1, 8), (300, 257, 520, 6), (129, 130, 131, 12)]
)
def test_ozaki_gemm_bitwise(dev, M, K, N, k):
    from trnblas_amd.hip import kernels

    A, B = inputs(M, K, N, seed=M + N)
    da, ea, b1 = kernels.ozaki_split(torch.from_numpy(A).to(dev), k, "row")
    db, eb, b2 = kernels.ozaki_split(torch.from_numpy(B).to(dev), k, "col")
    C = kernels.ozaki_gemm(da, ea, db, eb, M, N, k)
    torch.cuda.synchronize()
    assert int(b1) == 0 and int(b2) == 0
    want = oz.reference_gemm(A, B, k)
    # bitwise (no swap: the oracle swaps for N < 512 < M; compare unswapped)
    at, eA = oz.split_a(A, k)
    bt, eB = oz.split_b(B, k)
    hilo = oz.reference_from_digits(at, bt[:, :, :N])
    direct = oz.combine(hilo, eA, eB, k, M, N)
    got = C.cpu().numpy()
    assert np.array_equal(got.view(np.int64), direct.view(np.int64))
    if not (N < 512 and M > N):
        assert np.array_equal(got.view(np.int64), want.view(np.int64))


def test_ozaki_hilo_bitwise(dev):
    from trnblas_amd.hip import kernels

    A, B = inputs(100, 5000, 60, seed=11)
    k = 8
    da, _, _ = kernels.ozaki_split(torch.from_numpy(A).to(dev), k, "row")
    db, _, _ = kernels.ozaki_split(torch.from_numpy(B).to(dev), k, "col")
    hilo = kernels.ozaki_hilo(da, db, 100, 60, k).cpu().numpy()
    at, _ = oz.split_a(A, k)
    bt, _ = oz.split_b(B, k)
    want = oz.reference_from_digits(at, bt[:, :, :60])[:, :100, :60]
    assert np.array_equal(hilo.view(np.int32), want.view(np.int32))


@pytest.mark.parametrize("per", ["row", "col"])
@pytest.mark.parametrize("k", [3, 8])
def test_split_interleaved_layout(dev, per, k):
    # the interleaved digits are the plain split's digits with the k slices
    # of each 32-wide K chunk of a row side by side: (rows, Kp/32, k, 32)
    from trnblas_amd.hip import kernels

    rng = np.random.default_rng(40 + k)
    X = rng.standard_normal((150, 300)) * 10.0 ** rng.uniform(-20, 20, (150, 300))
    Xd = torch.from_numpy(X).to(dev)
    d, e, _ = kernels.ozaki_split(Xd, k, per)
    di, ei, bad = kernels.ozaki_split(Xd, k, per, interleaved=True)
    assert int(bad) == 0 and torch.equal(e, ei)
    _, rows, Kp = d.shape
    assert tuple(di.shape) == (rows, Kp * k)
    got = di.cpu().numpy().reshape(rows, Kp // 32, k, 32).transpose(2, 0, 1, 3).reshape(k, rows, Kp)
    assert np.array_equal(got, d.cpu().numpy())


@pytest.mark.parametrize(
    "M,K,N,k",
    [(64, 64, 64, 8), (130, 4100, 7, 8), (200, 9000, 31, 8), (300, 257, 520, 8), (1, 1, 1, 8),
     (65, 129, 63, 8), (200, 9000, 31, 1), (130, 4100, 70, 3), (300, 257, 520, 9),
     (200, 9000, 31, 10), (65, 129, 63, 10), (130, 4100, 70, 10), (33, 60000, 20, 10),
     (65, 129, 63, 11), (130, 4100, 70, 12), (33, 50000, 20, 12)],
)
def test_fast_gemm_interleaved_equals_plain(dev, M, K, N, k):
    # same digits, same int32 diagonal sums, same fp64 recombination order:
    # the interleaved-digit kernel must match the plain-layout one bit for bit
    # (K = 50000 at k = 12 and K = 60000 at k = 10 cross the int32 flush of the
    # diagonals; k = 10 runs its own two-workgroups-per-CU layout)
    from trnblas_amd.hip import kernels

    A, B = inputs(M, K, N, seed=M + 3 * N + k)
    Ad, Bd = torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev)
    da, ea, _ = kernels.ozaki_split(Ad, k, "row")
    db, eb, _ = kernels.ozaki_split(Bd, k, "col")
    dai, _, _ = kernels.ozaki_split(Ad, k, "row", interleaved=True)
    dbi, _, _ = kernels.ozaki_split(Bd, k, "col", interleaved=True)
    C1 = kernels.ozaki_gemm(da, ea, db, eb, M, N, k, fast=True)
    C2 = kernels.ozaki_gemm(dai, ea, dbi, eb, M, N, k, fast=True)
    assert torch.equal(C1, C2)
    C3 = kernels.ozaki_gemm(dbi, eb, dai, ea, N, M, k, fast=True, transpose_out=True)
    assert torch.equal(C1, C3) or bool(((C1 - C3).abs() <= 2.0**-50 * C1.abs()).all())
