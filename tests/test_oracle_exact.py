"""Pins of the independent fp64 judge (oracle/exact.py), CPU only."""

from fractions import Fraction

import numpy as np

from oracle.exact import inputs, max_cw, ref_exact


def test_exact_on_integer_products():
    rng = np.random.default_rng(1)
    A = rng.integers(-1000, 1000, (20, 300)).astype(np.float64)
    B = rng.integers(-1000, 1000, (300, 15)).astype(np.float64)
    assert np.array_equal(ref_exact(A, B), A @ B)  # exact in fp64 (< 2^53)


def test_close_to_rational_product():
    A, B = inputs(4, 50, 3, seed=7)
    R = ref_exact(A, B)
    for i in range(4):
        for j in range(3):
            exact = sum(Fraction(float(A[i, k])) * Fraction(float(B[k, j])) for k in range(50))
            assert abs(Fraction(float(R[i, j])) - exact) <= abs(exact) * Fraction(1, 2**51)


def test_max_cw_zero_for_exact_and_positive_for_perturbed():
    A, B = inputs(8, 40, 6, seed=2)
    ex = ref_exact(A, B)
    assert max_cw(ex, A, B, exact=ex) == 0.0
    assert max_cw(ex * (1 + 1e-12), A, B, exact=ex) > 0.0


def test_torch_form_bit_equal_to_numpy():
    """The device form (xp=torch) runs the same operations: same bits."""
    import torch

    for dist, shape, seed in (("logu4", (37, 500, 29), 3), ("normal", (16, 8192, 9), 4)):
        A, B = inputs(*shape, dist=dist, seed=seed)
        a = ref_exact(A, B)
        b = ref_exact(torch.from_numpy(A), torch.from_numpy(B), xp=torch).numpy()
        assert np.array_equal(a.view(np.int64), b.view(np.int64)), (dist, shape)
