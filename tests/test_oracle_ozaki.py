"""Pins of the Ozaki oracle (oracle/ozaki.py), CPU only.

Golden vectors written by the reference itself (tests/golden/ozaki_golden.npz,
tests/golden/make_golden.py) pin the digits, exponents, (hi, lo) and fp64
results bit for bit; invariants of the reference's own tests
(tests/test_ozaki.py:25-203 of the reference) pin the rest, against the
independent `oracle.exact.ref_exact`.
"""

import os

import numpy as np
import pytest

from oracle import ozaki as oz
from oracle.exact import inputs, max_cw

GOLD = os.path.join(os.path.dirname(__file__), "golden", "ozaki_golden.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD, allow_pickle=False)


@pytest.mark.parametrize("per", ["row", "col"])
@pytest.mark.parametrize("k", [1, 8, 12])
def test_split_matches_reference_golden(gold, per, k):
    X = gold["split_X"]
    d, e = oz.split(X, k, per=per, pad=(1, 1))
    assert np.array_equal(d, gold[f"split_{per}_k{k}_d"])
    assert np.array_equal(e, gold[f"split_{per}_k{k}_e"])


@pytest.mark.parametrize("c", range(5))
def test_reference_gemm_matches_reference_golden(gold, c):
    A, B, C = gold[f"gemm{c}_A"], gold[f"gemm{c}_B"], gold[f"gemm{c}_C"]
    k = int(gold[f"gemm{c}_k"])
    got = oz.reference_gemm(A, B, k)
    assert np.array_equal(got.view(np.int64), C.view(np.int64))


def test_hilo_matches_reference_golden(gold):
    A, B = gold["gemm0_A"], gold["gemm0_B"]
    at, _ = oz.split_a(A, 8)
    bt, _ = oz.split_b(B, 8)
    hilo = oz.reference_from_digits(at, bt[:, :, : B.shape[1]])
    assert np.array_equal(hilo.view(np.int32), gold["gemm0_hilo"].view(np.int32))


def test_schedule_known_answers(gold):
    assert [s for _, s, _ in oz.schedule(4, 3)] == list(gold["schedule_4_3_scales"])
    assert [d for d, _, _ in oz.schedule(4, 3)] == [3, 2, 1, 0]
    assert oz.n_products(8) == int(gold["n_products_8"]) == 36
    assert oz.exponent_offset(8) == int(gold["exponent_offset_8"]) == -61


@pytest.mark.parametrize("kt", [1, 7, 8, 31, 32, 33, 66, 100])
@pytest.mark.parametrize("d", [0, 1, 4, 7])
def test_diag_groups_cover_each_tile_once(kt, d):
    groups = oz.diag_groups(kt, d)
    flat = [(s, t, k0 + i) for g in groups for s, t, k0, n in g for i in range(n)]
    assert flat == [(s, d - s, j) for s in range(d + 1) for j in range(kt)]
    assert all(0 < sum(n for *_, n in g) <= oz.GROUP_TILES for g in groups)
    if kt >= oz.GROUP_TILES:
        assert all(len(g) == 1 for g in groups)
    else:
        per = oz.GROUP_TILES // kt
        assert all(len(g) == per for g in groups[:-1])


@pytest.mark.parametrize("per", ["row", "col"])
@pytest.mark.parametrize("k", [1, 3, 8, 12])
def test_split_digits_exact_and_bounded(per, k):
    rng = np.random.default_rng(0)
    X = rng.standard_normal((150, 300)) * np.logspace(-5, 5, 300)
    d, e = oz.split(X, k, per=per, pad=(128, 64))
    assert d.shape == (k, 256, 320)
    D = d.astype(np.float64)
    assert np.abs(D).max() <= 64
    assert not D[:, 150:].any() and not D[:, :, 300:].any()
    sc = np.ldexp(1.0, e - 6)
    sc = sc[:, None] if per == "row" else sc[None, :]
    rec = sum(D[s, :150, :300] * 2.0 ** (-7 * s) for s in range(k)) * sc
    bound = np.ldexp(1.0, e - 7 * k)
    bound = bound[:, None] if per == "row" else bound[None, :]
    assert (np.abs(rec - X) <= bound).all()


def test_split_extreme_zero_subnormal_rows():
    X = np.zeros((4, 300))
    X[0] = np.linspace(-1e300, 1e300, 300)
    X[1] = np.linspace(-1e-300, 1e-300, 300)
    X[2, 5] = 5e-324
    d, e = oz.split(X, 8, per="row", pad=(1, 1))
    D = d.astype(np.float64)
    rec = sum(D[s] * 2.0 ** (-7 * s) for s in range(8))
    for r in range(4):
        got = np.ldexp(rec[r], e[r] - 6)
        assert (np.abs(got - X[r]) <= np.ldexp(1.0, e[r] - 56)).all(), r
    assert not D[:, 3].any() and e[3] == 0


@pytest.mark.parametrize("shape", [(64, 64, 64), (37, 300, 53), (130, 4100, 7), (1, 1, 1)])
@pytest.mark.parametrize("k,tol", [(6, 2e-11), (7, 2e-13), (8, 1.5e-15)])
def test_reference_accuracy_vs_independent_exact(shape, k, tol):
    A, B = inputs(*shape)
    assert max_cw(oz.reference_gemm(A, B, k), A, B) <= tol


def test_reference_k1_is_exact_integer_product():
    rng = np.random.default_rng(3)
    A = rng.integers(-63, 64, (40, 5000)).astype(np.float64) * 2.0**-6
    B = rng.integers(-63, 64, (5000, 30)).astype(np.float64)
    assert np.array_equal(oz.reference_gemm(A, B, 1), A @ B)


def test_planted_twosum_order_mistake_is_caught(gold):
    # A plausible slip — folding the diagonals largest first — must fail the
    # golden comparison (the check is not vacuous).
    A, B, C = gold["gemm0_A"], gold["gemm0_B"], gold["gemm0_C"]
    orig = oz.schedule
    try:
        oz.schedule = lambda k, kt: list(reversed(orig(k, kt)))
        got = oz.reference_gemm(A, B, 8)
    finally:
        oz.schedule = orig
    assert not np.array_equal(got.view(np.int64), C.view(np.int64))


def test_plan_k_blocks():
    assert oz.plan_k_blocks(8192, 8) == [(0, 8192)]
    kb = oz.plan_k_blocks(1 << 20, 8)
    assert sum(n for _, n in kb) == 1 << 20 and all(n % 128 == 0 for _, n in kb)
    assert len(kb) > 1


@pytest.mark.parametrize("dist,k", [("normal", 8), ("logu4", 6), ("logu4", 8)])
def test_error_bound_holds_and_is_not_vacuous(dist, k):
    A, B = inputs(40, 700, 30, dist=dist, seed=9)
    C = oz.reference_gemm(A, B, k)
    from oracle.exact import ref_exact

    ex = ref_exact(A, B)
    bound = oz.error_bound(A, B, k)
    assert (np.abs(C - ex) <= bound).all()
    # one fewer slice breaks the k-slice bound somewhere (the bound is tight enough to see it)
    C_less = oz.reference_gemm(A, B, k - 2)
    assert not (np.abs(C_less - ex) <= bound).all()
