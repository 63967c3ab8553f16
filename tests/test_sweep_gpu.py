"""A seeded random sweep of the public Level-3 API on the GPU: shapes from 1
to a few thousand (ragged edges, tiny and long K, both layouts of every
operand, alpha / beta, broadcast batches), N(0, 1) and same-sign U(0, 1)
data, fp32 / bf16 / fp16, and gemm_fp64 in its three modes at 1..12 slices.

The sweep runs the HIP kernels (backend 'hip': no hipBLASLt route). Gates:
fp32 within 1e-6 |A||B| (+ |beta||C|) of fp64 (the north-star gate); 16-bit
within twice the output format's one rounding (bf16 2^-8, fp16 2^-10 of the
same magnitude, plus fp16's subnormal spacing, since a K = 1 product can fall
below fp16's range); SYRK exactly symmetric; gemm_fp64 within the reference's
truncation bound (oracle.ozaki.error_bound) and, for small exact-mode cases,
bit-equal to the reference arithmetic. The fixed case list keeps the sweep
deterministic."""

import random

import numpy as np
import pytest
import torch

import trnblas_amd as tb
from oracle import ozaki as oz

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-6, torch.bfloat16: 2.0**-8, torch.float16: 2.0**-10}
ABS = {torch.float32: 0.0, torch.bfloat16: 0.0, torch.float16: 2.0**-24}


def _excess(D, ref, den, dt):
    """Largest (|D - ref| - tol * den - abs floor); <= 0 passes."""
    if D.numel() == 0:
        return -1.0
    return float(((D.double() - ref).abs() - TOL[dt] * den - ABS[dt]).max())


def _dim(rng):
    r = rng.random()
    if r < 0.15:
        return rng.randint(1, 8)
    if r < 0.7:
        return rng.randint(9, 700)
    return rng.randint(700, 2500)


def _cases(seed, n):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        kind = rng.choice(["gemm", "gemm", "batched", "syrk", "syrk"])
        dt = rng.choice([torch.float32, torch.float32, torch.bfloat16, torch.float16])
        same = rng.random() < 0.4
        if kind == "gemm":
            p = (_dim(rng), _dim(rng), _dim(rng), rng.random() < 0.5, rng.random() < 0.5,
                 rng.choice([1.0, 2.0, -0.5]), rng.choice([0.0, 0.5, -1.0]))
        elif kind == "batched":
            b = rng.randint(1, 9)
            p = (rng.choice([b, 1]), rng.choice([b, 1]), rng.randint(1, 400), rng.randint(1, 400),
                 rng.randint(1, 900))
        else:
            p = (_dim(rng), _dim(rng), rng.random() < 0.5, rng.choice(["lower", "upper"]),
                 rng.choice([0.0, 0.5]))
        out.append((kind, dt, same, p))
    return out


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_level3_random_sweep(dev, seed, monkeypatch):
    from trnblas_amd.hip import dispatch

    monkeypatch.setattr(dispatch, "_backend", "hip")
    g = torch.Generator(device=dev).manual_seed(seed)

    def gen(*s, same=False):
        return torch.rand(*s, device=dev, generator=g) if same else torch.randn(*s, device=dev, generator=g)

    for kind, dt, same, p in _cases(seed, 60):
        if kind == "gemm":
            M, N, K, ta, tbb, alpha, beta = p
            A = (gen(K, M, same=same) if ta else gen(M, K, same=same)).to(dt)
            B = (gen(N, K, same=same) if tbb else gen(K, N, same=same)).to(dt)
            C = gen(M, N, same=same).to(dt) if beta else None
            D = tb.gemm(alpha, A, B, beta=beta, C=C, transA=ta, transB=tbb)
            Ae, Be = (A.T if ta else A).double(), (B.T if tbb else B).double()
            ref, den = alpha * (Ae @ Be), abs(alpha) * (Ae.abs() @ Be.abs())
            if C is not None:
                ref, den = ref + beta * C.double(), den + abs(beta) * C.double().abs()
        elif kind == "batched":
            bA, bB, M, N, K = p
            A, B = gen(bA, M, K, same=same).to(dt), gen(bB, K, N, same=same).to(dt)
            D = tb.batched_gemm(1.0, A, B)
            ref, den = A.double() @ B.double(), A.double().abs() @ B.double().abs()
        else:
            n, k, tr, uplo, beta = p
            A = (gen(k, n, same=same) if tr else gen(n, k, same=same)).to(dt)
            C = None
            if beta:
                C = gen(n, n, same=same)
                C = (C + C.T).to(dt)  # symmetric: no triangle rule applies
            D = tb.syrk(1.0, A, beta=beta, C=C, trans=tr, uplo=uplo)
            assert torch.equal(D, D.T), (kind, dt, p)
            op = (A.T if tr else A).double()
            ref, den = op @ op.T, op.abs() @ op.abs().T
            if C is not None:
                ref, den = ref + beta * C.double(), den + beta * C.double().abs()
        assert _excess(D, ref, den, dt) <= 0.0, (kind, dt, same, p)


@pytest.mark.parametrize("seed", [0, 1])
def test_gemm_fp64_random_sweep(dev, seed):
    rng = random.Random(100 + seed)
    for c in range(12):
        M, N, K = rng.randint(1, 300), rng.randint(1, 300), rng.randint(1, 2500)
        k, mode = rng.randint(1, 12), rng.choice(["fast", "exact", "crt"])
        r = np.random.default_rng(1000 * seed + c)
        A = r.uniform(-1, 1, (M, K)) * 2.0 ** np.round(r.normal(0, 4, (M, K)))
        B = r.uniform(-1, 1, (K, N))
        C = tb.gemm_fp64(torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev), slices=k, mode=mode)
        C = C.cpu().numpy()
        bound = oz.error_bound(A, B, k) + K * 2.0**-52 * (np.abs(A) @ np.abs(B))
        assert (np.abs(C - A @ B) <= bound).all(), (M, N, K, k, mode)
        if mode == "exact" and M * N * K <= 2_000_000:
            assert np.array_equal(C.view(np.int64), oz.reference_gemm(A, B, k).view(np.int64)), (M, N, K, k)
        if mode == "crt" and M * N <= 20_000:
            from oracle import ozaki_crt as oc

            assert np.array_equal(C.view(np.int64), oc.gemm_crt(A, B, k).view(np.int64)), (M, N, K, k)
