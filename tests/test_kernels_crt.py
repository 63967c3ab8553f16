"""The scheme-II (CRT) gemm_fp64 kernels on the GPU against the CPU oracle
(oracle/ozaki_crt.py), stage by stage and end to end, all bit for bit:
residues (integer arithmetic: exact), product residue planes (exact),
the recombination (the oracle restates its fp64 operations), the public
gemm_fp64(mode="crt"). Plus the k-slice error bound, long K (several K
blocks) and non-finite operands."""

import numpy as np
import pytest
import torch

import trnblas_amd as tb
from oracle import exact
from oracle import ozaki as oz
from oracle import ozaki_crt as oc

pytestmark = pytest.mark.gpu


def _unblock(P: np.ndarray, M: int, N: int) -> np.ndarray:
    """(nmod, nbm nbn 1024) blocked planes -> (nmod, M, N) (the layout of
    include/trnblas_hip.h, trnblas_hip_crt_gemm)."""
    nmod = P.shape[0]
    nbm, nbn = -(-M // 32), -(-N // 32)
    Q = P.reshape(nmod, nbm, nbn, 64, 16)
    bm, bn, l, e = np.meshgrid(np.arange(nbm), np.arange(nbn), np.arange(64), np.arange(16), indexing="ij")
    rows = 32 * bm + 8 * (e // 4) + 4 * (l // 32) + e % 4
    cols = 32 * bn + l % 32
    out = np.zeros((nmod, nbm * 32, nbn * 32), dtype=np.int8)
    out[:, rows, cols] = Q
    return out[:, :M, :N]


def _wide(M, K, N, seed, spread=12):
    rng = np.random.default_rng(seed)
    A = rng.uniform(-1, 1, (M, K)) * 2.0 ** np.round(rng.normal(0, spread / 3, (M, K)))
    B = rng.uniform(-1, 1, (K, N)) * 2.0 ** np.round(rng.normal(0, spread / 3, (K, N)))
    return A, B


@pytest.mark.parametrize("R,C", [(1, 1), (37, 300), (130, 64), (64, 130), (5, 1000)])
@pytest.mark.parametrize("k", [1, 8, 11, 12])
def test_crt_split_residues(dev, R, C, k):
    from trnblas_amd.hip import kernels

    A, _ = _wide(R, C, 1, seed=R + C + k)
    A[0, : min(3, C)] = 0.0
    if R > 2:
        A[2] = 0.0  # an all-zero row: exponent 0, residues 0
    n = oc.n_moduli(k, C)
    kp = -(-C // 64) * 64
    Ad = torch.from_numpy(A).to(dev)
    # rows of A (K = C)
    res, e, bad = kernels.crt_split(Ad, k, n, "row", kp)
    want, ew = oc.split(A, k, n, axis=1)
    got = kernels.crt_unblock(res).cpu().numpy()[:, :R]
    assert np.array_equal(got[:, :, :C], want) and not got[:, :, C:].any()
    assert np.array_equal(e.cpu().numpy(), ew) and int(bad) == 0
    # columns of A^T (the B role, written transposed): the same residues
    At = torch.from_numpy(np.ascontiguousarray(A.T)).to(dev)
    res2, e2, _ = kernels.crt_split(At, k, n, "col", kp)
    assert np.array_equal(kernels.crt_unblock(res2).cpu().numpy()[:, :R], got)
    assert np.array_equal(e2.cpu().numpy(), ew)


def test_crt_split_flags_non_finite(dev):
    from trnblas_amd.hip import kernels

    A = torch.randn(8, 70, dtype=torch.float64)
    A[3, 5] = float("inf")
    _, _, bad = kernels.crt_split(A.to(dev), 8, 16, "row", 128)
    assert int(bad) == 1
    _, _, bad = kernels.crt_split(A.T.contiguous().to(dev), 8, 16, "col", 128)
    assert int(bad) == 1


@pytest.mark.parametrize("M,K,N", [(1, 64, 1), (37, 300, 53), (300, 257, 200), (256, 128, 256), (513, 640, 97)])
def test_crt_gemm_planes(dev, M, K, N):
    from trnblas_amd.hip import kernels

    k = 8
    A, B = _wide(M, K, N, seed=M * N)
    n = oc.n_moduli(k, K)
    kp = -(-K // 64) * 64
    RA, _, _ = kernels.crt_split(torch.from_numpy(A).to(dev), k, n, "row", kp)
    RB, _, _ = kernels.crt_split(torch.from_numpy(B).to(dev), k, n, "col", kp)
    P = kernels.crt_gemm(RA, RB, M, N)
    got = _unblock(P.cpu().numpy(), M, N)
    ra, _ = oc.split(A, k, n, axis=1)
    rb, _ = oc.split(B, k, n, axis=0)
    assert np.array_equal(got, oc.planes(ra, rb))


@pytest.mark.parametrize("M,K,N,k", [(37, 300, 53, 8), (64, 1000, 40, 11), (100, 129, 300, 3), (33, 64, 1, 12)])
def test_crt_gemm_fp64_bit_equal_to_oracle(dev, M, K, N, k):
    A, B = _wide(M, K, N, seed=K + k)
    Ad, Bd = torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev)
    C = tb.gemm_fp64(Ad, Bd, slices=k, mode="crt").cpu().numpy()
    want = oc.gemm_crt(A, B, k)
    assert np.array_equal(C.view(np.int64), want.view(np.int64))
    # transposed views are split in their own layout: the same bits
    Ct = tb.gemm_fp64(Ad.mT.contiguous(), Bd.mT.contiguous(), slices=k, mode="crt", transA=True,
                      transB=True)
    assert np.array_equal(Ct.cpu().numpy().view(np.int64), want.view(np.int64))


@pytest.mark.parametrize("dist", ["normal", "logu4"])
@pytest.mark.parametrize("k", [4, 6, 8, 10])
def test_crt_within_k_slice_bound(dev, dist, k):
    A, B = exact.inputs(70, 900, 50, dist=dist, seed=10 + k)
    C = tb.gemm_fp64(torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev), slices=k, mode="crt")
    C = C.cpu().numpy()
    ex = exact.ref_exact(A, B)
    den = np.abs(A) @ np.abs(B)
    assert (np.abs(C - ex) <= oz.error_bound(A, B, k) + 900 * 2.0**-53 * den).all()
    assert exact.max_cw(C, A, B, exact=ex) <= exact.max_cw(oz.reference_gemm(A, B, k), A, B, exact=ex) * 1.01 + 2e-16


def test_crt_long_k_accumulates_blocks(dev):
    # K = 140000: three launches of K blocks (2^16 each), residues added mod m
    M, K, N, k = 40, 140000, 24, 8
    A, B = _wide(M, K, N, seed=3, spread=6)
    C = tb.gemm_fp64(torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev), slices=k, mode="crt")
    want = oc.gemm_crt(A, B, k)
    assert np.array_equal(C.cpu().numpy().view(np.int64), want.view(np.int64))


def test_crt_non_finite_falls_back(dev):
    A = torch.randn(20, 50, dtype=torch.float64)
    B = torch.randn(50, 30, dtype=torch.float64)
    A[4, 7] = float("nan")
    C = tb.gemm_fp64(A.to(dev), B.to(dev), mode="crt").cpu()
    want = A @ B
    assert torch.isnan(C[4]).all() and torch.allclose(C[:4], want[:4], rtol=1e-14, atol=0)
