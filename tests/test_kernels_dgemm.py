"""The fp64 MFMA GEMM (trnblas_hip_dgemm) and the diagonal-block inverse
(trnblas_hip_tri_inv_blocks) of the metric stage, on the GPU, against fp64
products computed on the host. Gate: componentwise
|D - D_ref| <= 1e-13 (|alpha| |A| |B| + |beta| |C|) (fp64 rounding of a
K-term sum is K 2^-53 in the worst case; the sums here are short enough)."""

import numpy as np
import pytest
import torch

from trnblas_amd.hip import _lib, kernels

pytestmark = pytest.mark.gpu


def _ref(A, B, alpha=1.0, beta=0.0, C=None):
    Ah, Bh = A.cpu().numpy(), B.cpu().numpy()
    ref = alpha * (Ah @ Bh)
    den = abs(alpha) * (np.abs(Ah) @ np.abs(Bh))
    if C is not None and beta != 0.0:
        Ch = np.broadcast_to(C.cpu().numpy(), ref.shape)
        ref = ref + beta * Ch
        den = den + abs(beta) * np.abs(Ch)
    return ref, den


def _cw(D, ref, den):
    den = np.where(den > 0, den, 1.0)
    return float((np.abs(D.cpu().numpy() - ref) / den).max())


def _mat(g, r, c, dev, trans=False):
    X = torch.randn((c, r) if trans else (r, c), generator=g, dtype=torch.float64).to(dev)
    return X.mT if trans else X


@pytest.mark.parametrize("M,N,K", [(1, 1, 2), (5, 7, 2), (130, 70, 64), (257, 129, 512),
                                   (64, 640, 128), (1024, 1024, 1024), (33, 17, 31)])
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False), (True, True)])
def test_dgemm_layouts(dev, M, N, K, ta, tb):
    g = torch.Generator().manual_seed(M * 7 + N * 3 + K + 2 * ta + tb)
    A, B = _mat(g, M, K, dev, ta), _mat(g, K, N, dev, tb)
    D = kernels.dgemm(A, B)
    ref, den = _ref(A, B)
    assert _cw(D, ref, den) <= 1e-13


def test_dgemm_epilogue_inplace_and_batched(dev):
    g = torch.Generator().manual_seed(3)
    A, B = _mat(g, 300, 256, dev), _mat(g, 256, 200, dev)
    C = _mat(g, 300, 200, dev)
    ref, den = _ref(A, B, -1.0, 1.0, C)
    kernels.dgemm(A, B, -1.0, 1.0, C, out=C)  # C -= A B in place
    assert _cw(C, ref, den) <= 1e-13
    # alpha / beta with a separate output, C not written
    C2 = _mat(g, 300, 200, dev)
    keep = C2.clone()
    D = kernels.dgemm(A, B, 0.5, -2.0, C2)
    ref, den = _ref(A, B, 0.5, -2.0, C2)
    assert _cw(D, ref, den) <= 1e-13 and torch.equal(C2, keep)
    # batched, with a broadcast operand and strided (as_strided) views
    A3 = torch.randn(5, 96, 160, generator=g, dtype=torch.float64).to(dev)
    B3 = torch.randn(1, 160, 72, generator=g, dtype=torch.float64).to(dev)
    D3 = kernels.dgemm(A3, B3)
    for i in range(5):
        ref, den = _ref(A3[i], B3[0])
        assert _cw(D3[i], ref, den) <= 1e-13
    big = torch.zeros(640, 640, dtype=torch.float64, device=dev)
    big[:] = torch.randn(640, 640, generator=g, dtype=torch.float64).to(dev)
    V = big.as_strided((2, 128, 128), (2 * 128 * 641, 640, 1), 128 * 640)  # blocks below the diagonal
    W = big.as_strided((2, 128, 128), (2 * 128 * 641, 640, 1), 0)
    Dv = kernels.dgemm(V, W)
    for i in range(2):
        ref, den = _ref(V[i], W[i])
        assert _cw(Dv[i], ref, den) <= 1e-13


def test_dgemm_odd_and_unaligned_operands(dev):
    g = torch.Generator().manual_seed(4)
    base = torch.randn(200 * 201 + 1, generator=g, dtype=torch.float64).to(dev)
    A = base[1 : 1 + 199 * 201].view(199, 201)[:, :199]  # 8-byte aligned, odd K, odd ld
    B = _mat(g, 199, 65, dev, trans=True)  # M/N-contiguous with an odd extent
    D = kernels.dgemm(A, B)
    ref, den = _ref(A, B)
    assert _cw(D, ref, den) <= 1e-13


@pytest.mark.parametrize("n", [300, 2048])  # 32- and 64-wide tiles
def test_dgemm_lower_and_triangular_operands(dev, n):
    g = torch.Generator().manual_seed(5)
    A = _mat(g, n, 128, dev)
    C = _mat(g, n, n, dev)
    upper_before = torch.triu(C, 1).clone()
    ref, den = _ref(A, A.mT, -1.0, 1.0, C)
    kernels.dgemm(A, A.mT, -1.0, 1.0, C, out=C, lower=True)
    lo = np.tril(np.ones((n, n), dtype=bool))
    err = np.abs(C.cpu().numpy() - ref) / np.where(den > 0, den, 1)
    assert err[lo].max() <= 1e-13
    assert torch.equal(torch.triu(C, 1), upper_before)  # the strict upper part is not written
    # triangular operands: the skipped blocks are exactly the zero ones
    for flags, a_tri, b_tri in [
        (_lib.TRI_A_LOWER, "lower", None),
        (_lib.TRI_A_UPPER, "upper", None),
        (_lib.TRI_B_LOWER, None, "lower"),
        (_lib.TRI_B_UPPER, None, "upper"),
        (_lib.TRI_A_LOWER | _lib.TRI_B_LOWER, "lower", "lower"),
    ]:
        X, Y = _mat(g, 384, 384, dev), _mat(g, 384, 256, dev)
        if a_tri:
            X = torch.tril(X) if a_tri == "lower" else torch.triu(X)
        if b_tri:
            Y = _mat(g, 384, 384, dev)
            Y = torch.tril(Y) if b_tri == "lower" else torch.triu(Y)
        D = kernels.dgemm(X, Y, tri=flags)
        ref, den = _ref(X, Y)
        assert _cw(D, ref, den) <= 1e-13, flags


@pytest.mark.parametrize("n", [1, 5, 128, 129, 300])
@pytest.mark.parametrize("upper", [False, True])
@pytest.mark.parametrize("unit", [False, True])
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_tri_inv_blocks(dev, n, upper, unit, dtype):
    g = torch.Generator().manual_seed(n + 2 * upper + unit)
    X = torch.randn(n, n, generator=g, dtype=torch.float64) / n + 2 * torch.eye(n, dtype=torch.float64)
    T = torch.triu(X) if upper else torch.tril(X)
    Tin = X.clone()  # the other triangle is garbage the kernel must not read
    Tin[torch.triu(torch.ones(n, n, dtype=torch.bool), 1) if not upper
        else torch.tril(torch.ones(n, n, dtype=torch.bool), -1)] = float("nan")
    if unit:
        T.fill_diagonal_(1.0)
        Tin.fill_diagonal_(float("nan"))
    D = kernels.tri_inv_blocks(Tin.to(dev, dtype), upper, unit).double().cpu()
    nb = kernels.TRI_NB
    tol = 1e-13 if dtype == torch.float64 else 2e-6
    for b in range(D.shape[0]):
        k0 = b * nb
        m = min(nb, n - k0)
        blk = T[k0 : k0 + m, k0 : k0 + m]
        Db = D[b]
        assert torch.equal(Db, torch.triu(Db) if upper else torch.tril(Db))
        assert (Db[:m, :m] @ blk - torch.eye(m, dtype=torch.float64)).abs().max() <= tol
        assert torch.equal(Db[m:, m:], torch.eye(nb - m, dtype=torch.float64))
        assert not Db[:m, m:].any() and not Db[m:, :m].any()
    # a transposed view is read through its strides
    Tv = Tin.to(dev, dtype).mT.contiguous().mT
    assert torch.equal(kernels.tri_inv_blocks(Tv, upper, unit).double().cpu(), D)
