"""Oracle: gemm_fp64 by Ozaki scheme II (CRT over int8 moduli) — TEST
INFRASTRUCTURE ONLY (see oracle/__init__.py).

The reference (trnblas/ozaki.py) multiplies fp64 matrices by splitting each
row of A / column of B into k 7-bit digits and summing the k (k + 1) / 2
digit products (ozaki.py:123-219, :337-455). Its precision knob `slices` = k
fixes how finely each operand is represented: to 2^(e - 7k) below its row /
column maximum 2^e (the truncation bound of ozaki.py:136-139).

Scheme II (Ozaki, Uchino and Imamura, "Ozaki Scheme II: A GEMM-oriented
emulation of floating-point matrix multiplication using an integer modular
technique", 2025) represents each operand to the same precision as one
integer instead of k digits, and multiplies the integers exactly through
the Chinese remainder theorem:

  1. A'_il = rint(a_il 2^(p - eA_i)), B'_lj = rint(b_lj 2^(p - eB_j)) with
     p = 7 k - 1 and eA_i / eB_j the frexp exponent of the row / column
     maximum (|A'| <= 2^p; the representation error is <= 2^(e - 7k), the
     k-slice truncation bound);
  2. for each modulus m_t of a fixed list of pairwise coprime m <= 256, the
     symmetric residues A'_t = A' mods m_t, B'_t = B' mods m_t (int8) and
     the int8 product P_t = A'_t B'_t mods m_t (exact: int32 sums);
  3. with enough moduli that M = prod m_t > 2 K 2^(2p) + 2, the exact
     integer C' = A' B' (|C'| <= K 2^(2p) < M / 2) is the unique balanced
     value with those residues: Garner's mixed-radix digits
     v_1 = r_1, v_t = ((r_t - sum_{s<t} v_s P_{s-1}) P_{t-1}^-1) mods m_t,
     C' = v_1 + m_1 (v_2 + m_2 (v_3 + ...)) evaluated by Horner with fp64
     fma from the top, two digits per step;
  4. C = C' 2^(eA_i + eB_j - 2p).

The error against the exact product is the operand truncation alone (no
dropped digit products), so it stays within the k-slice bound of
`oracle.ozaki.error_bound`; the work is one int8 GEMM per modulus (C5, k = 11:
22 GEMMs where the digit split runs 66).

Functions:
* `MODULI`, `bits`, `n_moduli`: the moduli list and how many a call uses;
* `split` : exponents and the integer operand A' (fp64 integers), residues;
* `planes`: the per-modulus product residues (exact int64);
* `garner`: the mixed-radix digits (exact integers);
* `horner_fp64`: the kernel's fp64 evaluation of C' (fma emulated exactly
  with Python integers), and `reconstruct_exact` (Python-int C');
* `gemm_crt`: the whole product, the kernels' arithmetic op for op.

Pinned by tests/test_oracle_ozaki_crt.py: pairwise coprimality and the
modulus-count rule against Python-int products; residues against Python's
`%` on the exact integers; Garner against random integers in the balanced
range (every value comes back) and against brute-force Python-int products
A' B'; the fp64 Horner within (G - 1) / 2 + 1 ulp of the exact C' (G
fma steps); the
end-to-end result within the k-slice bound of the near-exact product and
more accurate than the digit split at equal k.
"""

from __future__ import annotations

import math

import numpy as np

# Pairwise coprime moduli <= 256, largest first; 256 first makes the balanced
# mixed-radix range exactly [-M/2, M/2 - 1].
MODULI = (256, 255, 253, 251, 247, 241, 239, 233, 229, 227, 223, 217, 211, 199, 197, 193,
          191, 181, 179, 173, 167, 163, 157, 151, 149, 139, 137, 131, 127, 113, 109, 107)  # fmt: skip


def bits(slices: int) -> int:
    """Operand precision p of `slices` 7-bit digits: 6 bits for the first
    digit (|digit| <= 64), 7 for each further one (ozaki.py:127-139)."""
    return 7 * slices - 1


def n_moduli(slices: int, K: int) -> int:
    """The fewest leading MODULI whose product M >= 2 K 2^(2p) + 2, so every
    |C'| <= K 2^(2p) lies in the balanced range [-M/2, M/2 - 1]."""
    p = bits(slices)
    need = 2 * max(K, 1) * (1 << (2 * p)) + 2
    M = 1
    for n, m in enumerate(MODULI, 1):
        M *= m
        if M >= need:
            return n
    raise ValueError(f"no modulus set for slices={slices}, K={K}")


def smod(x, m: int):
    """The balanced residue of integer x modulo m: [-m/2, m/2) for even m,
    [-(m-1)/2, (m-1)/2] for odd m."""
    r = np.mod(x, m)
    return np.where(r >= m - m // 2, r - m, r)


def exponents(X: np.ndarray, axis: int) -> np.ndarray:
    """frexp exponent of the largest |x| along `axis` (0 for an all-zero
    line): every |x| < 2^e."""
    amax = np.abs(X).max(axis=axis)
    return np.where(amax > 0, np.frexp(amax)[1], 0).astype(np.int64)


def integer_operand(X: np.ndarray, p: int, axis: int):
    """(X', e): X' = rint(x 2^(p - e)) per row (axis=1) or column (axis=0),
    as fp64 integers (exact: |X'| <= 2^p)."""
    X = np.asarray(X, dtype=np.float64)
    e = exponents(X, axis)
    sh = (p - e)[:, None] if axis == 1 else (p - e)[None, :]
    return np.rint(np.ldexp(X, sh)), e


def residues(Xi: np.ndarray, m: int) -> np.ndarray:
    """Balanced residues of the fp64 integers Xi (|Xi| < 2^90) mod m, int8."""
    a = np.abs(Xi)
    big = a >= 2.0**53
    E = np.frexp(np.where(big, a, 1.0))[1]
    sh = np.where(big, E - 53, 0).astype(np.int64)
    mant = np.ldexp(a, -sh).astype(np.int64)  # exact: < 2^53
    pw = np.array([pow(2, int(s), m) for s in range(64)], dtype=np.int64)
    r = (mant % m) * pw[sh] % m
    r = np.where(Xi < 0, -r, r)
    return smod(r, m).astype(np.int8)


def split(X: np.ndarray, slices: int, nmod: int, axis: int):
    """(res (nmod, *X.shape) int8, e): residues of the integer operand."""
    Xi, e = integer_operand(X, bits(slices), axis)
    return np.stack([residues(Xi, m) for m in MODULI[:nmod]]), e


def planes(RA: np.ndarray, RB: np.ndarray) -> np.ndarray:
    """P_t = RA_t @ RB_t mods m_t (int8), RA (nmod, M, K), RB (nmod, K, N)."""
    out = []
    for t in range(RA.shape[0]):
        P = RA[t].astype(np.int64) @ RB[t].astype(np.int64)
        out.append(smod(P, MODULI[t]).astype(np.int8))
    return np.stack(out)


def garner(R: np.ndarray) -> np.ndarray:
    """Balanced mixed-radix digits v (nmod, ...) of the value with residues
    R (nmod, ...) mod MODULI[:nmod]: value = sum_t v_t prod_{s<t} m_s."""
    n = R.shape[0]
    v = np.zeros(R.shape, dtype=np.int64)
    for t in range(n):
        m = MODULI[t]
        acc = np.zeros(R.shape[1:], dtype=np.int64)
        P = 1
        for s in range(t):
            acc += v[s] * (P % m)
            P *= MODULI[s]
        inv = pow(P % m, -1, m) if t else 1
        v[t] = smod((R[t].astype(np.int64) - acc) % m * inv, m)
    return v


def reconstruct_exact(v: np.ndarray) -> np.ndarray:
    """C' = sum_t v_t prod_{s<t} m_s as Python ints (object array)."""
    out = np.zeros(v.shape[1:], dtype=object)
    P = 1
    for t in range(v.shape[0]):
        out = out + v[t].astype(object) * P
        P *= MODULI[t]
    return out


def horner_fp64(v: np.ndarray) -> np.ndarray:
    """The kernel's evaluation of sum_t v_t prod_{s<t} m_s in fp64: digits
    paired into radix-(m_2g m_2g+1) digits V_g = v_2g + m_2g v_2g+1 (exact,
    |V_g| < 2^15), then H = V_top and H = fma(H, m_2g m_2g+1, V_g) down to
    g = 0, one rounding per step (emulated exactly: H is an integer-valued
    double, so the fma is the correctly rounded integer H mu + V, which
    Python's int -> float conversion computes)."""
    n = v.shape[0]
    G = (n + 1) // 2
    V = [v[2 * g] + (MODULI[2 * g] * v[2 * g + 1] if 2 * g + 1 < n else 0) for g in range(G)]
    H = V[G - 1].astype(np.float64)
    for g in range(G - 2, -1, -1):
        mu = MODULI[2 * g] * MODULI[2 * g + 1]
        Hi = np.vectorize(lambda h: int(h), otypes=[object])(H)
        H = (Hi * mu + V[g].astype(object)).astype(np.float64)
    return H


def gemm_crt(A: np.ndarray, B: np.ndarray, slices: int = 8, nmod: int | None = None) -> np.ndarray:
    """op-for-op model of the device's scheme-II product (fp64 (M, N))."""
    A = np.asarray(A, dtype=np.float64)
    B = np.asarray(B, dtype=np.float64)
    K = A.shape[1]
    p = bits(slices)
    n = n_moduli(slices, K) if nmod is None else nmod
    RA, eA = split(A, slices, n, axis=1)
    RB, eB = split(B, slices, n, axis=0)
    v = garner(planes(RA, RB))
    H = horner_fp64(v)
    return np.ldexp(H, (eA[:, None] + eB[None, :] - 2 * p))


def exact_integer_product(A, B, slices: int):
    """The exact C' = A' B' with Python ints (brute force, tiny inputs)."""
    p = bits(slices)
    Ai, _ = integer_operand(A, p, 1)
    Bi, _ = integer_operand(B, p, 0)
    Ao = np.vectorize(lambda x: int(x), otypes=[object])(Ai)
    Bo = np.vectorize(lambda x: int(x), otypes=[object])(Bi)
    return Ao.dot(Bo)


def modulus_product(n: int) -> int:
    return math.prod(MODULI[:n])
