"""Pins of the scheme-II (CRT) gemm_fp64 oracle (oracle/ozaki_crt.py), CPU only."""

import math

import numpy as np
import pytest

from oracle import exact
from oracle import ozaki as oz
from oracle import ozaki_crt as oc


def test_moduli_pairwise_coprime_and_int8():
    for i, a in enumerate(oc.MODULI):
        assert 2 <= a <= 256
        for b in oc.MODULI[i + 1 :]:
            assert math.gcd(a, b) == 1, (a, b)
    assert oc.MODULI[0] == 256  # the balanced range is then exactly [-M/2, M/2 - 1]


@pytest.mark.parametrize("k,K", [(1, 1), (1, 8192), (8, 8192), (11, 8192), (12, 1 << 17), (8, 3)])
def test_modulus_count_is_minimal(k, K):
    p = oc.bits(k)
    n = oc.n_moduli(k, K)
    bound = K * (1 << (2 * p))  # |A' B'| <= K 2^(2p)
    assert oc.modulus_product(n) >= 2 * bound + 2
    assert n == 1 or oc.modulus_product(n - 1) < 2 * bound + 2


def test_modulus_counts_at_c5():
    assert oc.n_moduli(8, 8192) == 16 and oc.n_moduli(11, 8192) == 22


def test_residues_match_python_ints():
    rng = np.random.default_rng(3)
    x = np.rint(rng.standard_normal(4000) * 2.0 ** rng.integers(0, 85, 4000))
    x[:6] = [0.0, 1.0, -1.0, 2.0**84, -(2.0**84) + 2**40, 127.0]
    for m in oc.MODULI:
        r = oc.residues(x, m)
        want = [int(xi) % m for xi in x]
        assert all((int(ri) - w) % m == 0 for ri, w in zip(r, want))
        lo, hi = -(m // 2), m - m // 2 - 1
        assert r.min() >= lo and r.max() <= hi


def test_integer_operand_precision():
    # |X'| <= 2^p and X' 2^(e-p) is x to within 2^(e-p-1) (the k-slice truncation)
    rng = np.random.default_rng(4)
    X = rng.standard_normal((7, 50)) * 2.0 ** rng.integers(-20, 20, (7, 50))
    for k in (1, 5, 8, 11):
        p = oc.bits(k)
        Xi, e = oc.integer_operand(X, p, axis=1)
        assert np.abs(Xi).max() <= 2.0**p
        err = np.abs(np.ldexp(Xi, (e - p)[:, None]) - X)
        assert (err <= np.ldexp(1.0, (e - 7 * k)[:, None])).all()


def test_garner_recovers_every_balanced_value():
    rng = np.random.default_rng(5)
    for n in (1, 2, 5, 16, 22, 32):
        M = oc.modulus_product(n)
        vals = [-(M // 2), M // 2 - 1, 0, 1, -1] + [int(rng.integers(-(2**62), 2**62)) * int(rng.integers(1, 2**40)) % M - M // 2 for _ in range(200)]
        R = np.array([[((x + m // 2) % m) - m // 2 if m % 2 == 0 else ((x + (m - 1) // 2) % m) - (m - 1) // 2
                       for x in vals] for m in oc.MODULI[:n]], dtype=np.int64)  # fmt: skip
        v = oc.garner(R)
        got = oc.reconstruct_exact(v)
        assert list(got) == vals, n


def test_planes_and_garner_give_the_exact_integer_product():
    # brute force: A' B' with Python ints equals the CRT reconstruction
    rng = np.random.default_rng(6)
    A = rng.standard_normal((5, 37)) * 2.0 ** rng.integers(-30, 30, (5, 37))
    B = rng.standard_normal((37, 4)) * 2.0 ** rng.integers(-30, 30, (37, 4))
    for k in (1, 3, 8, 11, 12):
        n = oc.n_moduli(k, 37)
        RA, _ = oc.split(A, k, n, axis=1)
        RB, _ = oc.split(B, k, n, axis=0)
        got = oc.reconstruct_exact(oc.garner(oc.planes(RA, RB)))
        want = oc.exact_integer_product(A, B, k)
        assert (got == want).all(), k
    # one modulus too few wraps around for some element (the count is needed)
    k = 8
    n = oc.n_moduli(k, 37)
    A2 = np.full((2, 37), 0.9999)
    B2 = np.full((37, 2), 0.9999)
    RA, _ = oc.split(A2, k, n - 1, axis=1)
    RB, _ = oc.split(B2, k, n - 1, axis=0)
    bad = oc.reconstruct_exact(oc.garner(oc.planes(RA, RB)))
    assert (bad != oc.exact_integer_product(A2, B2, k)).any()


@pytest.mark.parametrize("n", [16, 22, 32])
def test_horner_close_to_the_exact_integer(n):
    # each of the G - 1 fma steps (G = ceil(n / 2) paired digits) rounds once,
    # by at most half an ulp of a partial value that the later steps scale up
    # to the final one: |H - C'| <= (G - 1) / 2 + 1 ulp of C'
    rng = np.random.default_rng(7 + n)
    M = oc.modulus_product(n)
    vals = [int(rng.integers(-(2**62), 2**62)) * int(rng.integers(1, 2**62)) * int(rng.integers(1, 2**62))
            * int(rng.integers(1, 2**62)) % M - M // 2 for _ in range(1000)]  # fmt: skip
    vals += [1, -1, 0, 2**100 + 1, -(2**120) + 12345, M // 2 - 1, -(M // 2)]
    R = np.array([oc.smod(np.array([x % m for x in vals], dtype=np.int64), m) for m in oc.MODULI[:n]])
    H = oc.horner_fp64(oc.garner(R))
    G = (n + 1) // 2
    worst = 0.0
    for h, x in zip(H, vals):
        f = float(x)
        if f == 0.0:
            assert h == 0.0
            continue
        worst = max(worst, abs(h - f) / np.spacing(abs(f)))
    assert worst <= (G - 1) / 2 + 1, worst


@pytest.mark.parametrize("dist", ["normal", "logu4"])
@pytest.mark.parametrize("k", [3, 6, 8, 11])
def test_gemm_crt_within_k_slice_bound_and_tighter_than_digits(dist, k):
    A, B = exact.inputs(23, 300, 17, dist=dist, seed=k)
    C = oc.gemm_crt(A, B, k)
    ex = exact.ref_exact(A, B)
    K = A.shape[1]
    den = np.abs(A) @ np.abs(B)
    assert (np.abs(C - ex) <= oz.error_bound(A, B, k) + K * 2.0**-53 * den).all()
    # no dropped digit products: at equal k at least as accurate as the split
    e_crt = exact.max_cw(C, A, B, exact=ex)
    e_dig = exact.max_cw(oz.reference_gemm(A, B, k), A, B, exact=ex)
    assert e_crt <= max(e_dig, 2e-16), (e_crt, e_dig)


def test_gemm_crt_integer_operands_exact():
    # small integers with a common row / column scale: the product is exact
    rng = np.random.default_rng(8)
    A = rng.integers(-63, 64, (9, 400)).astype(np.float64)
    B = rng.integers(-63, 64, (400, 7)).astype(np.float64)
    A[:, 0] = 63
    B[0] = 63
    assert np.array_equal(oc.gemm_crt(A, B, 1), A @ B)


def test_zero_rows_and_columns():
    A = np.zeros((3, 10))
    A[1, 4] = 3.5
    B = np.zeros((10, 2))
    B[4, 1] = -2.0
    C = oc.gemm_crt(A, B, 8)
    assert np.array_equal(C, A @ B)
