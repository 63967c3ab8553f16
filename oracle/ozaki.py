"""Oracle: the Ozaki fp64-class GEMM of trnblas (trnblas/ozaki.py), restated.

Test infrastructure only (see oracle/__init__.py).

The arithmetic is the reference's, step for step, because `gemm_fp64`'s
contract is bit-exactness against `ozaki.reference_gemm`
(trnblas/level3.py:137-171): the same digit split, the same group cut of each
diagonal of slice products, the same fp32 TwoSum order, the same fp64
recombination, the same narrow-N swap and K blocking. Digits are returned as
int8 (the reference stores the same small integers in bf16).

Pinned by (tests/test_oracle_ozaki.py):
* golden vectors written by the reference itself (tests/golden/ozaki_*.npz,
  made by tests/golden/make_golden.py in the build container): digits,
  exponents, (hi, lo) and the fp64 result, compared bit for bit;
* the split invariants of the reference tests (test_ozaki.py:25-54):
  integer digits, |d| <= 64, zero padding, reconstruction within
  2^(e - 7k), extreme / zero / subnormal rows;
* schedule known answers (test_ozaki.py:138-142) and the cover-once
  invariant (:115-129);
* accuracy against the independent `oracle.exact.ref_exact` at
  k = 6/7/8 (:179-187) and k = 1 integer exactness (:197-203).
"""

from __future__ import annotations

import math

import numpy as np

SLICE_BITS = 7  # ozaki.py:42
TILE_K = 128  # ozaki.py:43
GROUP_TERMS = 4096  # ozaki.py:44
GROUP_TILES = GROUP_TERMS // TILE_K  # ozaki.py:45
MIN_SLICES, MAX_SLICES, DEFAULT_SLICES = 1, 12, 8  # ozaki.py:46-48
BLOCK_BYTES = 1 << 31  # ozaki.py:462
SWAP_N = 512  # ozaki.py:476
LAUNCH_M = LAUNCH_N = 1024  # ozaki.py:482-483


def check_slices(slices) -> int:
    """ozaki.py:51-58."""
    if isinstance(slices, bool) or not isinstance(slices, (int, np.integer)):
        raise TypeError(f"slices must be an int, got {type(slices).__name__}")
    k = int(slices)
    if not MIN_SLICES <= k <= MAX_SLICES:
        raise ValueError(f"slices must be in [{MIN_SLICES}, {MAX_SLICES}], got {k}")
    return k


def n_products(k: int) -> int:
    """ozaki.py:61-63: slice pairs (s, t) with s + t <= k - 1."""
    return k * (k + 1) // 2


def round_up(n: int, m: int) -> int:
    return -(-n // m) * m


def exponent_offset(k: int) -> int:
    """ozaki.py:373-375."""
    return -2 * (SLICE_BITS - 1) - SLICE_BITS * (k - 1)


def split(X: np.ndarray, k: int, per: str = "col", pad=(TILE_K, 1)):
    """ozaki.py:123-219. Digits int8 (k, Rp, Cp) and int64 exponents of the
    rows (per="row") or columns (per="col") of the finite fp64 matrix X."""
    k = check_slices(k)
    X = np.ascontiguousarray(X, dtype=np.float64)
    R, C = X.shape
    Rp, Cp = round_up(max(R, 1), pad[0]), round_up(max(C, 1), pad[1])
    digits = np.zeros((k, Rp, Cp), dtype=np.int8)
    axis = 1 if per == "row" else 0
    n = R if per == "row" else C
    if R == 0 or C == 0:
        return digits, np.zeros(n, dtype=np.int64)
    amax = np.abs(X).max(axis=axis)
    e = np.frexp(amax)[1].astype(np.int64)  # amax < 2^e; 0 -> 0
    shift = (SLICE_BITS - 1) - e
    # One power-of-two factor when every shift is a normal exponent, else two
    # (a global choice over all rows / columns, ozaki.py:185-188).
    if shift.max() <= 1023 and shift.min() >= -1022:
        factors = [np.ldexp(1.0, shift)]
    else:
        factors = [np.ldexp(1.0, shift // 2), np.ldexp(1.0, shift - shift // 2)]
    if per == "row":
        factors = [f[:, None] for f in factors]
    else:
        factors = [f[None, :] for f in factors]
    rem = X * factors[0]
    for f in factors[1:]:
        rem = rem * f
    radix = float(1 << SLICE_BITS)
    for s in range(k):
        if s:
            rem = rem * radix
        d = np.rint(rem)
        if s + 1 < k:
            rem = rem - d
        digits[s, :R, :C] = d.astype(np.int8)
    return digits, e


def diag_groups(kt: int, d: int) -> list:
    """ozaki.py:337-355: the groups of diagonal d (pairs (s, d - s)) for kt
    K tiles per slice, as lists of runs (s, t, first tile, tiles)."""
    pairs = [(s, d - s) for s in range(d + 1)]
    if kt >= GROUP_TILES:
        out = []
        for s, t in pairs:
            for k0 in range(0, kt, GROUP_TILES):
                out.append([(s, t, k0, min(GROUP_TILES, kt - k0))])
        return out
    per = GROUP_TILES // kt
    return [[(s, t, 0, kt) for s, t in pairs[i : i + per]] for i in range(0, len(pairs), per)]


def schedule(k: int, kt: int) -> list:
    """ozaki.py:358-365: [(d, scale, groups)] with d = k-1 down to 0."""
    return [
        (d, float(2 ** (SLICE_BITS * (k - 1 - d))), diag_groups(kt, d))
        for d in range(k - 1, -1, -1)
    ]


def n_groups(k: int, kt: int) -> int:
    """ozaki.py:368-370."""
    return sum(len(g) for _, _, g in schedule(k, kt))


def two_sum32(hi: np.ndarray, lo: np.ndarray, p: np.ndarray):
    """ozaki.py:378-386: fp32 Knuth TwoSum of hi + p, its error added to lo,
    in the reference's operation order."""
    f32 = np.float32
    hi, lo, p = hi.astype(f32), lo.astype(f32), p.astype(f32)
    s = hi + p
    v = s - hi
    w = s - v
    err = (hi - w) + (p - v)
    return s, lo + err


def reference_from_digits(at: np.ndarray, b: np.ndarray) -> np.ndarray:
    """ozaki.py:389-415. at (k, Kp, Mp) and b (k, Kp, N) digit stacks (K
    major) -> float32 (2, Mp, N) = (hi, lo): exact integer group sums, each
    times its diagonal's power-of-two scale, folded by `two_sum32` in
    schedule order starting from (0, 0)."""
    k, Kp, Mp = at.shape
    if Kp % TILE_K:
        raise ValueError(f"Kp must be a multiple of {TILE_K}")
    A = at.astype(np.float64)
    B = b.astype(np.float64)
    hi = np.zeros((Mp, b.shape[2]), dtype=np.float32)
    lo = np.zeros_like(hi)
    for _d, scale, groups in schedule(k, Kp // TILE_K):
        for grp in groups:
            acc = np.zeros((Mp, b.shape[2]), dtype=np.float64)
            for s, t, k0, nt in grp:
                r0, r1 = k0 * TILE_K, (k0 + nt) * TILE_K
                acc += A[s, r0:r1].T @ B[t, r0:r1]  # integers < 2^24: exact
            hi, lo = two_sum32(hi, lo, (acc * scale).astype(np.float32))
    return np.stack([hi, lo])


def combine(hilo: np.ndarray, eA, eB, k: int, M: int, N: int) -> np.ndarray:
    """ozaki.py:418-455: fp64 (hi + lo) 2^(eA_i + eB_j + offset), exact
    power-of-two scaling (one rounding of the product when it is
    subnormal)."""
    if M == 0 or N == 0:
        return np.zeros((M, N))
    v = hilo[0, :M, :N].astype(np.float64) + hilo[1, :M, :N].astype(np.float64)
    ea = np.asarray(eA[:M], dtype=np.int64) + exponent_offset(k)
    eb = np.asarray(eB[:N], dtype=np.int64)
    if max(abs(int(ea.max())), abs(int(ea.min()))) < 900 and max(
        abs(int(eb.max())), abs(int(eb.min()))
    ) < 900:
        return v * np.ldexp(1.0, ea)[:, None] * np.ldexp(1.0, eb)[None, :]
    return np.ldexp(v, ea[:, None] + eb[None, :])


def plan_k_blocks(Kp: int, k: int, limit: int = BLOCK_BYTES) -> list:
    """The K blocking of ozaki.py:486-511 (`plan`): one block unless a
    1024-row launch over all of K would pass `limit`. M / N blocks do not
    change the arithmetic and are not restated."""
    cap = limit // (2 * k)
    Kb = Kp if Kp * 1024 <= cap else max(TILE_K, (cap // 1024) // TILE_K * TILE_K)
    return [(i, min(Kb, Kp - i)) for i in range(0, Kp, Kb)]


def split_a(A: np.ndarray, k: int):
    """ozaki.py:310-319 values: A (M, K) split by rows -> K-major digits
    (k, Kp, Mp), exponents (M,)."""
    d, e = split(A, k, per="row", pad=(TILE_K, TILE_K))
    return np.ascontiguousarray(d.transpose(0, 2, 1)), e


def split_b(B: np.ndarray, k: int):
    """ozaki.py:322-329 values: B (K, N) split by columns -> K-major digits
    (k, Kp, Np), exponents (N,)."""
    d, e = split(B, k, per="col", pad=(TILE_K, TILE_K))
    return d, e


def reference_gemm(A: np.ndarray, B: np.ndarray, k: int = DEFAULT_SLICES) -> np.ndarray:
    """ozaki.py:514-595 (`run` with `reference_launch`): fp64 A @ B by the
    device arithmetic, bit for bit. Finite fp64 A (M, K), B (K, N)."""
    k = check_slices(k)
    A = np.asarray(A, dtype=np.float64)
    B = np.asarray(B, dtype=np.float64)
    M, K = A.shape
    N = B.shape[1]
    if M == 0 or N == 0 or K == 0:
        return np.zeros((M, N))
    at, eA = split_a(A, k)
    bt, eB = split_b(B, k)
    swap = N < SWAP_N and M > N  # ozaki.py:546-547: C^T = B^T A^T
    if swap:
        at, eA, bt, eB, M, N = bt, eB, at, eA, N, M
    C = None
    for k0, kb in plan_k_blocks(at.shape[1], k):
        hilo = reference_from_digits(at[:, k0 : k0 + kb], bt[:, k0 : k0 + kb, :N])
        part = combine(hilo, eA, eB, k, M, N)
        C = part if C is None else C + part
    return C.T.copy() if swap else C


def digits_exact_bound(e: np.ndarray, k: int) -> np.ndarray:
    """|x - 2^(e - 6) sum_s d_s 2^(-7 s)| <= 2^(e - 7 k) (ozaki.py:136-139)."""
    return np.ldexp(1.0, np.asarray(e) - SLICE_BITS * k)


def log2_ceil(x: float) -> int:
    return int(math.ceil(math.log2(x)))


def error_bound(A, B, k: int, absA_absB=None, xp=np):
    """The a-priori componentwise bound of the k-slice product. With
    t = 2^-7k, |digit| <= 64 (so slice s of a row is at most 2^(eA - 7s)), the
    truncation |x - sum_s slice_s| <= 2^(e - 7k) (ozaki.py:123-139), and the
    pairs s + t >= k that the schedule drops (ozaki.py:337-365):

      |C - AB|_ij <= t (2^eA_i sum_k |b_kj| + sum_k |a_ik| 2^eB_j)
                     + 1.01 (k - 1 + t) t 2^(eA_i + eB_j) K
                     + 2^-46 (|A||B|)_ij

    The last term is the observed floor of the fp32 (hi, lo) pair (the
    reference measures 2e-16 .. 3e-16 of |A||B| at k = 8, ozaki.py:28-34).
    Works on numpy arrays or (xp=torch) device tensors."""
    if xp is np:
        A = np.asarray(A, dtype=np.float64)
        B = np.asarray(B, dtype=np.float64)
        aA, aB = np.abs(A), np.abs(B)
        eA = np.frexp(aA.max(axis=1))[1].astype(np.float64)
        eB = np.frexp(aB.max(axis=0))[1].astype(np.float64)
        ra, cb = np.exp2(eA)[:, None], np.exp2(eB)[None, :]
        rows, cols = aA.sum(axis=1)[:, None], aB.sum(axis=0)[None, :]
        AB = aA @ aB if absA_absB is None else absA_absB
    else:
        aA, aB = A.abs(), B.abs()
        eA = xp.frexp(aA.amax(dim=1))[1].double()
        eB = xp.frexp(aB.amax(dim=0))[1].double()
        ra, cb = xp.exp2(eA)[:, None], xp.exp2(eB)[None, :]
        rows, cols = aA.sum(dim=1)[:, None], aB.sum(dim=0)[None, :]
        AB = aA @ aB if absA_absB is None else absA_absB
    t = 2.0 ** (-SLICE_BITS * k)
    K = A.shape[1]
    return t * (ra * cols + rows * cb) + 1.01 * (k - 1 + t) * t * ra * cb * K + 2.0**-46 * AB
