"""Oracle: the DF-MP2 pair energy of trnblas, restated.

Test infrastructure only (see oracle/__init__.py).

  E = sum_{i,j < nocc} sum_{a,b < nvir} T_ab (2 T_ab - T_ba) / (e_i + e_j - v_a - v_b),
  T = B_i B_j^T,  B (nocc, nvir, naux).

* `pair_energy_f64`      the closed form in float64 by the symmetric walk
                         (i <= j, weight 2 off the diagonal: e_ij = e_ji) —
                         the parity judge (north star: relative 1e-6);
* `pair_energy_f64_full` the same over all ordered pairs (no symmetry used);
* `batched_pair_cpu`     the reference's CPU/torch path, an nocc^2 loop
                         accumulated in B's dtype (dispatch.py:2514-2533);
* `chunked_pair_cpu`     the aten route: chunked GEMM + torch reduction
                         (dispatch.py:2706-2728) — also the *unfused GPU
                         baseline* when given device tensors;
* `energy_reduction_cpu` the example's default energy step
                         (examples/df_mp2.py:51-99);
* `mp2_energy_cpu`       the reduction of a precomputed T_flat
                         (dispatch.py:1440-1453, `_torch_mp2_energy`);
* `fused_pair_cpu`       one pair (dispatch.py:3027-3046);
* `pair_sym_dims`        the reference's window / weights of the per-row walk
                         (dispatch.py:2648-2677).

Pinned by tests/test_oracle_pair_energy.py: the symmetric walk equals the
full ordered loop (independent summation), brute-force per-element loops on
tiny shapes, B = 0 -> 0, rank-one B with a closed-form energy, invariance
under permuting virtual orbitals (with eps_vir), e_ij = e_ji, and the
reference's known window weights (test_native_dispatch.py:1080-1090).
"""

from __future__ import annotations

import torch


def _denom(ei, ej, ev):
    return ei + ej - ev[:, None] - ev[None, :]


def pair_energy_f64(B, eps_occ, eps_vir) -> float:
    B = B.detach().double().cpu()
    eo = eps_occ.detach().double().cpu()
    ev = eps_vir.detach().double().cpu()
    nocc = B.shape[0]
    total = 0.0
    for i in range(nocc):
        # all j >= i at once: T_ij for j in i..nocc-1
        T = torch.einsum("ap,jbp->jab", B[i], B[i:])
        D = eo[i] + eo[i:, None, None] - ev[None, :, None] - ev[None, None, :]
        e = (T * (2.0 * T - T.transpose(1, 2)) / D).sum(dim=(1, 2))
        w = torch.full_like(e, 2.0)
        w[0] = 1.0
        total += float((w * e).sum())
    return total


def pair_energy_f64_full(B, eps_occ, eps_vir) -> float:
    B = B.detach().double().cpu()
    eo = eps_occ.detach().double().cpu()
    ev = eps_vir.detach().double().cpu()
    total = 0.0
    for i in range(B.shape[0]):
        for j in range(B.shape[0]):
            T = B[i] @ B[j].T
            total += float((T * (2.0 * T - T.T) / _denom(eo[i], eo[j], ev)).sum())
    return total


def pair_energies_f64(Bi, Bj, eps_i, eps_j, eps_vir, pairs) -> torch.Tensor:
    """Unweighted e_p for explicit pairs, float64 (host)."""
    Bi, Bj = Bi.detach().double().cpu(), Bj.detach().double().cpu()
    ei, ej = eps_i.detach().double().cpu(), eps_j.detach().double().cpu()
    ev = eps_vir.detach().double().cpu()
    out = torch.empty(len(pairs), dtype=torch.float64)
    for p, (i, j) in enumerate(pairs):
        T = Bi[i] @ Bj[j].T
        out[p] = (T * (2.0 * T - T.T) / _denom(ei[i], ej[j], ev)).sum()
    return out


def batched_pair_cpu(B, eps_occ, eps_vir, rows=None) -> torch.Tensor:
    """dispatch.py:2514-2533: the nocc^2 loop, summed in B's dtype. rows: the
    rows i to loop over (default all; a subset gives a timing sample)."""
    e = torch.zeros((), dtype=B.dtype, device=B.device)
    nocc = B.shape[0]
    for i in range(nocc) if rows is None else rows:
        for j in range(nocc):
            T = B[i] @ B[j].T
            D = float(eps_occ[i]) + float(eps_occ[j]) - eps_vir.unsqueeze(1) - eps_vir.unsqueeze(0)
            e = e + (T * (2.0 * T - T.T) / D).sum()
    return e


def chunked_pair_cpu(B, eps_occ, eps_vir, mem_budget_bytes: int = 1_500_000_000):
    """dispatch.py:2706-2728: T for an i-chunk at once (one GEMM), then the
    torch reduction; the chunk keeps T under `mem_budget_bytes`."""
    nocc, nvir, naux = B.shape
    i_block = max(1, min(nocc, int(mem_budget_bytes // (4 * nvir * nocc * nvir))))
    flat = B.reshape(nocc * nvir, naux)
    eo2 = eps_occ.view(nocc, 1, 1, 1) + eps_occ.view(1, nocc, 1, 1)
    ev2 = eps_vir.view(1, 1, nvir, 1) + eps_vir.view(1, 1, 1, nvir)
    e = torch.zeros((), dtype=B.dtype, device=B.device)
    for i0 in range(0, nocc, i_block):
        i1 = min(i0 + i_block, nocc)
        T = (flat[i0 * nvir : i1 * nvir] @ flat.T).reshape(i1 - i0, nvir, nocc, nvir)
        T = T.permute(0, 2, 1, 3)
        e = e + (T * (2.0 * T - T.transpose(-2, -1)) / (eo2[i0:i1] - ev2)).sum()
    return e


def energy_reduction_cpu(B, eps_occ, eps_vir, mem_budget_bytes: int = 1_500_000_000) -> float:
    """examples/df_mp2.py:51-99 (default path): T_chunk = B_chunk @ B_flat^T
    through `gemm(transB=True)`, then the torch reduction."""
    nocc, nvir, naux = B.shape
    i_block = max(1, min(nocc, int(mem_budget_bytes // (4 * nvir * nocc * nvir))))
    flat = B.reshape(nocc * nvir, naux).contiguous()
    eo2 = eps_occ.view(nocc, 1, 1, 1) + eps_occ.view(1, nocc, 1, 1)
    ev2 = eps_vir.view(1, 1, nvir, 1) + eps_vir.view(1, 1, 1, nvir)
    e = torch.zeros((), dtype=B.dtype, device=B.device)
    for i0 in range(0, nocc, i_block):
        i1 = min(i0 + i_block, nocc)
        T = torch.matmul(flat[i0 * nvir : i1 * nvir], flat.T)
        T = T.reshape(i1 - i0, nvir, nocc, nvir).permute(0, 2, 1, 3)
        e = e + (T * (2.0 * T - T.transpose(-2, -1)) / (eo2[i0:i1] - ev2)).sum()
    return float(e)


def mp2_energy_cpu(T_flat, eps_occ_chunk, eps_occ_full, eps_vir) -> torch.Tensor:
    """dispatch.py:1440-1453 (`_torch_mp2_energy`)."""
    ic, nocc, nvir = eps_occ_chunk.shape[0], eps_occ_full.shape[0], eps_vir.shape[0]
    T = T_flat.reshape(ic, nvir, nocc, nvir).permute(0, 2, 1, 3)
    D = (
        eps_occ_chunk.view(ic, 1, 1, 1)
        + eps_occ_full.view(1, nocc, 1, 1)
        - eps_vir.view(1, 1, nvir, 1)
        - eps_vir.view(1, 1, 1, nvir)
    )
    return (T * (2.0 * T - T.transpose(-2, -1)) / D).sum()


def fused_pair_cpu(b_i, b_j, eps_i: float, eps_j: float, eps_vir) -> torch.Tensor:
    """dispatch.py:3027-3046: one pair."""
    T = b_i @ b_j.T
    D = eps_i + eps_j - eps_vir.unsqueeze(1) - eps_vir.unsqueeze(0)
    return (T * (2.0 * T - T.T) / D).sum()


def pair_sym_dims(nocc: int, nvir: int, naux: int) -> dict:
    """dispatch.py:2648-2677: padded sizes and the per-d weights of the
    per-row window j = i + d (mod nocc), d = 0 .. nocc // 2 (padded to an even
    count with weight-0 entries)."""
    rup = lambda n: -(-n // 128) * 128  # noqa: E731
    half = nocc // 2
    nd = half + 1
    nd_pad = nd + (nd % 2)
    w = [2.0] * nd_pad
    w[0] = 1.0
    if half > 0 and nocc % 2 == 0:
        w[half] = 1.0
    for d in range(nd, nd_pad):
        w[d] = 0.0
    nv, na = rup(nvir), rup(naux)
    return dict(
        nvir_pad=nv,
        naux_pad=na,
        nd_pad=nd_pad,
        weights=w,
        sbuf_bytes=4 * nv * (2 * (na // 128) + nv // 128),
        row_flop=2.0 * nd * nv * nv * na,
    )
