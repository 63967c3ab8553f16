"""Oracle: an independent near-correctly-rounded fp64 matrix product.

Test infrastructure only (see oracle/__init__.py).

Restates the accuracy judge of the reference's Ozaki tests
(tests/_ozaki_ref.py:16-56): an fp64 Ozaki split with slices narrow enough
(b = floor((55 - log2 K) / 2) bits, k = ceil(80 / b) slices) that every host
fp64 slice GEMM is exact, products summed smallest first with Neumaier
compensation. It shares no code with `oracle.ozaki` (different split,
different accumulation), so it can judge it.

Pinned by tests/test_oracle_exact.py: integer-valued inputs whose product is
exactly representable (ref_exact must equal it exactly), products with
known closed forms, and agreement with the exact rational product
(fractions.Fraction) on small random matrices to within one ulp.
"""

from __future__ import annotations

import math

import numpy as np


def ref_exact(A, B, xp=np):
    """The near-correctly-rounded product of A (M, K) and B (K, N).

    xp=np: numpy arrays on the host. xp=torch: fp64 tensors on any device,
    the same operations in the same order. Every slice product is exact in
    any fp64 GEMM, whatever its summation order or blocking: a piece is
    q 2^(e - c) with |q| <= 2^(b-1), so each term of a slice product's row i,
    column j is an integer multiple of 2^(eA_i + eB_j - c_s - c_t) below
    2^(2b-2) of that unit, and the K terms and every partial sum stay below
    K 2^(2b-2) <= 2^53 units. The elementwise Neumaier steps are the same
    IEEE operations on both, so the two give the same bits (checked by the
    GPU test that uses the device form)."""
    if xp is np:
        A = np.asarray(A, dtype=np.float64)
        B = np.asarray(B, dtype=np.float64)
    K = A.shape[1]
    b = math.floor((55 - math.log2(max(K, 2))) / 2)
    k = math.ceil(80 / b)

    def pieces(X, axis):
        if xp is np:
            amax = np.abs(X).max(axis=axis, keepdims=True)
            nz = amax > 0
            e = np.where(nz, np.ceil(np.log2(np.where(nz, amax, 1.0))), 0.0)
            rem = X * np.exp2(-e)
        else:
            amax = X.abs().amax(dim=axis, keepdim=True)
            nz = amax > 0
            e = xp.where(nz, xp.ceil(xp.log2(xp.where(nz, amax, xp.ones_like(amax)))),
                         xp.zeros_like(amax))
            rem = X * xp.exp2(-e)
        out = []
        for s in range(k):
            width = (b - 1) if s == 0 else b
            scaled = rem * 2.0**width
            q = xp.round(scaled) if xp is not np else np.rint(scaled)
            rem = scaled - q
            out.append(q * xp.exp2(e - ((b - 1) + b * s)))
        return out

    Ap, Bp = pieces(A, 1), pieces(B, 0)
    order = sorted(
        [(s, t) for s in range(k) for t in range(k) if s + t <= k - 1], key=lambda st: -sum(st)
    )
    total = comp = None
    for s, t in order:
        P = Ap[s] @ Bp[t]
        if total is None:
            total, comp = P, xp.zeros_like(P)
            continue
        nxt = total + P
        big = xp.abs(total) >= xp.abs(P)
        comp += xp.where(big, (total - nxt) + P, (P - nxt) + total)
        total = nxt
        del P, nxt, big
    return total + comp


def max_cw(C, A, B, exact=None) -> float:
    """max |C - C_exact| / (|A| |B|), componentwise (tests/_ozaki_ref.py:51-56)."""
    A = np.asarray(A, dtype=np.float64)
    B = np.asarray(B, dtype=np.float64)
    den = np.abs(A) @ np.abs(B)
    den = np.where(den > 0, den, 1.0)
    ex = ref_exact(A, B) if exact is None else exact
    return float((np.abs(np.asarray(C, dtype=np.float64) - ex) / den).max())


def inputs(M, K, N, dist="normal", seed=0):
    """Seeded fp64 A (M, K), B (K, N): "normal" N(0, 1), or "logu4" (entries
    spread over 10^+-4), as tests/_ozaki_ref.py:59-68."""
    rng = np.random.default_rng(seed)
    if dist == "normal":
        return rng.standard_normal((M, K)), rng.standard_normal((K, N))
    A = rng.standard_normal((M, K)) * 10.0 ** rng.uniform(-4, 4, (M, K))
    B = rng.standard_normal((K, N)) * 10.0 ** rng.uniform(-4, 4, (K, N))
    return A, B
