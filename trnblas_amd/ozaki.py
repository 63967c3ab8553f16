"""fp64-class GEMM by Ozaki splitting on gfx950 int8 MFMA — the host half.

MI355X counterpart of trnblas/ozaki.py. The schedule constants and the
pure functions that define the arithmetic contract (`check_slices`,
`n_products`, `diag_groups`, `schedule`, `n_groups`, `exponent_offset`,
`plan`) keep the reference's semantics (trnblas/ozaki.py:42-63, :337-375,
:462-511). The data path differs: the split, the slice products and the
recombination all run on the device (`run_device`), from the fp64 operands
in HBM, in three kernel launches per operand pair — no host digit arrays,
no host combine, no launch blocking below 2 GiB.

Bit-exactness: `run_device` equals the reference's `ozaki.reference_gemm`
bit for bit (same digits, same group cut, same fp32 TwoSum order, same fp64
combine, same narrow-N swap and K blocking). The CPU restatement that
checks this lives in `oracle/ozaki.py` (test infrastructure); this module
has no CPU arithmetic path.
"""

from __future__ import annotations

import os

import numpy as np
import torch

SLICE_BITS = 7
TILE_K = 128
GROUP_TERMS = 4096
GROUP_TILES = GROUP_TERMS // TILE_K
MIN_SLICES = 1
MAX_SLICES = 12
DEFAULT_SLICES = 8
BLOCK_BYTES = 1 << 31
SWAP_N = 512


class OzakiNonFinite(Exception):
    """An operand of gemm_fp64 holds inf / nan (the digits cannot represent it)."""


def check_slices(slices) -> int:
    """`slices` as an int in [MIN_SLICES, MAX_SLICES] (ozaki.py:51-58)."""
    if isinstance(slices, bool) or not isinstance(slices, (int, np.integer)):
        raise TypeError(f"slices must be an int, got {type(slices).__name__}")
    k = int(slices)
    if not MIN_SLICES <= k <= MAX_SLICES:
        raise ValueError(f"slices must be in [{MIN_SLICES}, {MAX_SLICES}], got {k}")
    return k


def n_products(slices: int) -> int:
    """Slice GEMMs per product: pairs (s, t) with s + t <= slices - 1."""
    return slices * (slices + 1) // 2


def _round_up(n: int, m: int) -> int:
    return -(-n // m) * m


def diag_groups(kt: int, d: int) -> list:
    """Groups of diagonal d for kt K tiles per slice, in accumulation order
    (ozaki.py:337-355): runs (s, t, first tile, tiles) of at most GROUP_TILES
    tiles; with kt >= GROUP_TILES each pair is cut on its own, otherwise
    GROUP_TILES // kt whole pairs share a group."""
    pairs = [(s, d - s) for s in range(d + 1)]
    if kt >= GROUP_TILES:
        return [
            [(s, t, k0, min(GROUP_TILES, kt - k0))]
            for s, t in pairs
            for k0 in range(0, kt, GROUP_TILES)
        ]
    per = GROUP_TILES // kt
    return [[(s, t, 0, kt) for s, t in pairs[i : i + per]] for i in range(0, len(pairs), per)]


def schedule(slices: int, kt: int) -> list:
    """[(d, scale, groups)], diagonals smallest first (ozaki.py:358-365)."""
    return [
        (d, float(2 ** (SLICE_BITS * (slices - 1 - d))), diag_groups(kt, d))
        for d in range(slices - 1, -1, -1)
    ]


def n_groups(slices: int, kt: int) -> int:
    return sum(len(g) for _, _, g in schedule(slices, kt))


def exponent_offset(slices: int) -> int:
    """C = (hi + lo) * 2^(eA_i + eB_j + exponent_offset(slices))."""
    return -2 * (SLICE_BITS - 1) - SLICE_BITS * (slices - 1)


def k_block(Kp: int, slices: int, limit: int = BLOCK_BYTES) -> int:
    """The K block of the reference's launch plan (ozaki.py:486-511): Kp
    itself unless a 1024-row launch over all of K would pass `limit` (K of
    about 2^17 or more), else the largest multiple of TILE_K that fits; the
    last block may be shorter. The reference's M / N blocks change nothing in
    the arithmetic (each block's (hi, lo) chains are the same), so only the
    K block is computed."""
    cap = limit // (2 * check_slices(slices))
    if Kp * 1024 <= cap:
        return Kp
    return max(TILE_K, (cap // 1024) // TILE_K * TILE_K)


# The reference's launch caps (ozaki.py:470-481): Trainium compile time grows
# with a launch's whole problem, so its launches are capped at 1024 x 1024
# outputs. The int8 kernels here need no cap; the names stay for callers.
LAUNCH_M = 1024
LAUNCH_N = 1024


def _cuts(total: int, step: int) -> list:
    return [(i, min(step, total - i)) for i in range(0, total, step)]


def plan(Mp: int, Kp: int, N: int, slices: int, limit: int = BLOCK_BYTES,
         max_m: int = LAUNCH_M, max_n: int = LAUNCH_N):
    """The reference's launch blocks (m_blocks, k_blocks, n_blocks), each
    [(start, size)] (ozaki.py:484-511), for callers of that interface: every
    launch at most max_m x max_n outputs with its operands (2 k Kb Mb,
    2 k Kb Nb bytes) and result (8 Mb Nb bytes) within `limit`. Here only
    the K block changes the arithmetic (`k_block`, which `run_device` uses):
    the M / N blocks of one launch compute the same (hi, lo) chains, so the
    kernels cover all of M and N in one launch."""
    k = check_slices(slices)
    cap = limit // (2 * k)
    kb = k_block(Kp, k, limit)
    mb = max(TILE_K, min(Mp, max_m // TILE_K * TILE_K, (cap // kb) // TILE_K * TILE_K))
    nb = max(1, min(N, max_n, cap // kb))
    if 8 * mb * nb > limit:
        nb = max(1, min(nb, limit // (8 * mb)))
    return _cuts(Mp, mb), _cuts(Kp, kb), _cuts(N, nb)


def split_device(X: torch.Tensor, slices: int, per: str, interleaved: bool = False,
                 check: bool = True):
    """Device digits of `ozaki.split(X, slices, per, pad=(128, 128))`:
    int8 (k, rows, Kp) with K contiguous, where rows are X's rows (per="row")
    or columns (per="col"), and int32 exponents. interleaved: the same digits
    as (rows, Kp * k), the slices of each 32-wide K chunk side by side.
    check: raise OzakiNonFinite for a non-finite X (one device-to-host read);
    otherwise return (digits, exps, flag) with the 0-d device flag, the
    digits being undefined when it is set."""
    from .hip import kernels

    d, e, bad = kernels.ozaki_split(X, slices, per, interleaved)
    if not check:
        return d, e, bad
    if int(bad):  # one small device-to-host read
        raise OzakiNonFinite()
    return d, e


def _digits_of(X: torch.Tensor, k: int, want: str, interleaved: bool = False):
    """Digits, exponents and non-finite flag for the operand role `want`
    ("rows of A" = per-row split of A, "cols of B" = per-column split of B).
    A transposed view is split in its own layout (as ozaki.split_a / split_b
    do), so no fp64 copy is made."""
    if want == "A":  # A (M, K): per row, digits (k, M, Kp)
        if X.mT.is_contiguous() and not X.is_contiguous():
            return split_device(X.mT, k, "col", interleaved, False)  # A^T (K, M) by columns
        return split_device(X.contiguous(), k, "row", interleaved, False)
    # B (K, N): per column, digits (k, N, Kp)
    if X.mT.is_contiguous() and not X.is_contiguous():
        return split_device(X.mT, k, "row", interleaved, False)  # B^T (N, K) by rows
    return split_device(X.contiguous(), k, "col", interleaved, False)


MODES = ("fast", "exact", "crt")


def default_mode() -> str:
    """How gemm_fp64 multiplies: TRNBLAS_OZAKI_MODE = "fast" (default: the
    reference's digits and slice products, each diagonal of slice pairs
    summed exactly in int32, all diagonals recombined in fp64; within the
    reference's truncation bound), "exact" (the reference's groups and fp32
    TwoSum order: bit-equal to `ozaki.reference_gemm`) or "crt" (Ozaki scheme
    II: each operand rounded to the precision of `slices` digits as one
    integer, the integer product exact by the Chinese remainder theorem over
    int8 moduli; within the same bound, with no dropped digit products, in
    n_moduli GEMMs instead of slices (slices + 1) / 2)."""
    return check_mode(os.environ.get("TRNBLAS_OZAKI_MODE", "fast").strip().lower())


def check_mode(mode: str | None) -> str:
    if mode is None:
        return default_mode()
    if mode not in MODES:
        raise ValueError(f"Ozaki mode must be one of {MODES}; got {mode!r}")
    return mode


def _residues_of(X: torch.Tensor, k: int, nmod: int, kp: int, want: str):
    """Residues (nmod, rows, kp) of the operand role `want` ("A": rows of A,
    "B": columns of B); a transposed view is split in its own layout."""
    from .hip import kernels

    if want == "A":
        if X.mT.is_contiguous() and not X.is_contiguous():
            return kernels.crt_split(X.mT, k, nmod, "col", kp)
        return kernels.crt_split(X.contiguous(), k, nmod, "row", kp)
    if X.mT.is_contiguous() and not X.is_contiguous():
        return kernels.crt_split(X.mT, k, nmod, "row", kp)
    return kernels.crt_split(X.contiguous(), k, nmod, "col", kp)


def _run_crt(A: torch.Tensor, B: torch.Tensor, k: int, C: torch.Tensor) -> torch.Tensor:
    """Scheme II on the device: residues of both operands, one int8 GEMM per
    modulus (one launch), the CRT recombination into C."""
    from .hip import kernels

    M, K = A.shape
    N = B.shape[1]
    nmod = kernels.crt_moduli(k, K)
    kp = _round_up(K, kernels.CRT_KP)
    RA, eA, bad_a = _residues_of(A, k, nmod, kp, "A")
    RB, eB, bad_b = _residues_of(B, k, nmod, kp, "B")
    P = kernels.crt_gemm(RA, RB, M, N)
    del RA, RB
    kernels.crt_combine(P, eA, eB, M, N, k, out=C)
    if int(bad_a | bad_b):  # one small device-to-host read
        raise OzakiNonFinite()
    return C


def run_device(
    A: torch.Tensor, B: torch.Tensor, slices: int = DEFAULT_SLICES, mode: str | None = None
) -> torch.Tensor:
    """C = A @ B in fp64 by Ozaki splitting, on the device. A (M, K), B (K, N)
    fp64 device tensors (views allowed). mode "exact" is bit-equal to the
    reference's `ozaki.reference_gemm(A, B, slices)`; "fast" has the same
    digits and products with an fp64 recombination (see default_mode)."""
    from .hip import kernels

    k = check_slices(slices)
    mode = check_mode(mode)
    M, K = A.shape
    N = B.shape[1]
    C = torch.empty((M, N), dtype=torch.float64, device=A.device)
    if M == 0 or N == 0:
        return C
    if K == 0:
        return C.zero_()
    if mode == "crt":
        return _run_crt(A, B, k, C)
    fast = mode == "fast"
    # the fast schedule reads the digits interleaved (a row's k slices of a
    # 32-wide K chunk side by side)
    il = fast
    # the non-finite flags are read once, after the GEMM (no stall between the
    # launches; a GEMM on undefined digits stays in bounds and is discarded)
    da, ea, bad_a = _digits_of(A, k, "A", il)
    db, eb, bad_b = _digits_of(B, k, "B", il)
    Kp = da.shape[1] // k if il else da.shape[2]
    kb = k_block(Kp, k) if mode == "exact" else Kp
    if N < SWAP_N and M > N:  # C^T = B^T A^T (ozaki.py:546-547): B's digits first
        kernels.ozaki_gemm(db, eb, da, ea, N, M, k, kb=kb, out=C, transpose_out=True, fast=fast)
    else:
        kernels.ozaki_gemm(da, ea, db, eb, M, N, k, kb=kb, out=C, fast=fast)
    if int(bad_a | bad_b):  # one small device-to-host read
        raise OzakiNonFinite()
    return C
