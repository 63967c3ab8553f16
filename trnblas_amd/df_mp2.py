"""The DF-MP2 energy step (and the config-4 chain) on trnblas_amd.

The MI355X counterpart of the energy step of examples/df_mp2.py:
* `energy_reduction` — the example's default path (df_mp2.py:51-99):
  chunked `gemm(B_chunk, B_flat, transB=True)` + torch reduction;
* `energy_reduction_batched_pair` — its `--batched-pair-energy` path
  (df_mp2.py:131-144): one fused HIP launch for every pair;
* `half_transform` / `df_mp2_chain_energy` — the config-4 chain: the two
  half-transforms of a P-major 3-center tensor as two one-launch batched
  GEMMs writing B directly in the (nocc, nvir, naux) layout the fused energy
  kernel reads, then the fused energy;
* seeded synthetic inputs of the benchmark configurations.
"""

from __future__ import annotations

import math

import torch

from . import level3
from .hip import dispatch as _d


def energy_reduction(B, eps_occ, eps_vir, *, mem_budget_bytes: int = 1_500_000_000) -> float:
    """E = sum_{ijab} T_ijab (2 T_ijab - T_ijba) / D_ijab by chunked GEMM
    (one `gemm(..., transB=True)` per i-chunk, B_flat^T read in place) and a
    torch reduction (examples/df_mp2.py:51-99)."""
    nocc, nvir, naux = B.shape
    i_block = max(1, min(nocc, int(mem_budget_bytes // (4 * nvir * nocc * nvir))))
    flat = B.reshape(nocc * nvir, naux)
    eo2 = eps_occ.view(nocc, 1, 1, 1) + eps_occ.view(1, nocc, 1, 1)
    ev2 = eps_vir.view(1, 1, nvir, 1) + eps_vir.view(1, 1, 1, nvir)
    e = torch.zeros((), dtype=B.dtype, device=B.device)
    for i0 in range(0, nocc, i_block):
        i1 = min(i0 + i_block, nocc)
        T = level3.gemm(1.0, flat[i0 * nvir : i1 * nvir], flat, transB=True)
        T = T.reshape(i1 - i0, nvir, nocc, nvir).permute(0, 2, 1, 3)
        e = e + (T * (2.0 * T - T.transpose(-2, -1)) / (eo2[i0:i1] - ev2)).sum()
    return float(e)


def energy_reduction_batched_pair(B, eps_occ, eps_vir) -> float:
    """The fused pair energy (examples/df_mp2.py:131-144)."""
    return float(_d.nki_batched_pair_energy(B, eps_occ, eps_vir))


def half_transform(eri: torch.Tensor, C_occ: torch.Tensor, C_vir: torch.Tensor) -> torch.Tensor:
    """B[i, a, P] = sum_{mu, nu} C_occ[mu, i] C_vir[nu, a] eri[P, mu, nu] for a
    P-major 3-center tensor eri (naux, nao, nao).

    Two one-launch batched GEMMs, no transposed copies:
      T1[P] = C_occ^T @ eri[P]                  (naux, nocc, nao)
      B[i]  = C_vir^T @ T1[:, i, :]^T           (nocc, nvir, naux)
    The second reads T1 through a strided view (batch stride nao, the
    transposed operand read in place), so B comes out aux-contiguous."""
    naux, nao, _ = eri.shape
    nocc, nvir = C_occ.shape[1], C_vir.shape[1]
    T1 = level3.batched_gemm(1.0, C_occ.mT.unsqueeze(0).expand(naux, nocc, nao), eri)
    T1v = T1.permute(1, 2, 0)  # (nocc, nao, naux) view: T1v[i] = T1[:, i, :]^T
    return level3.batched_gemm(1.0, C_vir.mT.unsqueeze(0).expand(nocc, nvir, nao), T1v)


def df_mp2_chain_energy(eri, C_occ, C_vir, eps_occ, eps_vir, timings: dict | None = None):
    """Config 4: half-transforms into B, then the fused pair energy."""
    sync = _d._device_synchronize
    import time

    t0 = time.perf_counter()
    B = half_transform(eri, C_occ, C_vir)
    sync()
    t1 = time.perf_counter()
    e = _d.nki_batched_pair_energy(B, eps_occ, eps_vir)
    e = float(e)
    t2 = time.perf_counter()
    if timings is not None:
        timings.update(half=t1 - t0, energy=t2 - t1)
    return e


def chain_flops(nao: int, nocc: int, nvir: int, naux: int) -> dict:
    """Algorithmic flops of the config-4 chain (symmetric pair count)."""
    return dict(
        half1=2.0 * naux * nocc * nao * nao,
        half2=2.0 * nocc * nvir * nao * naux,
        energy=nocc * (nocc + 1) / 2 * 2.0 * nvir * nvir * naux,
    )


# ── seeded synthetic inputs of the benchmark configurations ─────────────────
#
# All draws on the host in fp64 from torch.Generator().manual_seed(seed), in
# the listed order, then cast and copied to the device (same values on any
# machine). Config 4's 17 GB 3-center tensor is drawn on the device instead
# (seeded device generator): a host draw of 4.3 G normals takes minutes.


def config1_inputs(device, seed: int = 0):
    """C1: A (2048 x 2048, stored K x M for transA), B, C_init ~ N(0, 1)."""
    g = torch.Generator().manual_seed(seed)
    A = torch.randn(2048, 2048, generator=g, dtype=torch.float64)
    B = torch.randn(2048, 2048, generator=g, dtype=torch.float64)
    C = torch.randn(2048, 2048, generator=g, dtype=torch.float64)
    return tuple(x.float().to(device) for x in (A, B, C))


def config2_inputs(device, seed_syrk: int = 1, seed_batched: int = 2):
    """C2a: A 4096 x 8192 and symmetric C 4096 x 4096 (N(0,1) entries);
    C2b: A (64, 512, 2048), B (64, 2048, 512)."""
    g = torch.Generator().manual_seed(seed_syrk)
    A = torch.randn(4096, 8192, generator=g, dtype=torch.float64)
    X = torch.randn(4096, 4096, generator=g, dtype=torch.float64)
    C = torch.tril(X) + torch.tril(X, diagonal=-1).mT
    g2 = torch.Generator().manual_seed(seed_batched)
    Ab = torch.randn(64, 512, 2048, generator=g2, dtype=torch.float64)
    Bb = torch.randn(64, 2048, 512, generator=g2, dtype=torch.float64)
    return tuple(x.float().to(device) for x in (A, C, Ab, Bb))


def pair_inputs(nocc: int, nvir: int, naux: int, device="cpu", seed: int = 3):
    """C3 rules at any size: B = 0.05 N(0, 1), eps_occ ~ U(-1.5, -0.3),
    eps_vir ~ U(0.1, 3.0)."""
    g = torch.Generator().manual_seed(seed)
    B = 0.05 * torch.randn(nocc, nvir, naux, generator=g, dtype=torch.float64)
    eo = -1.5 + 1.2 * torch.rand(nocc, generator=g, dtype=torch.float64)
    ev = 0.1 + 2.9 * torch.rand(nvir, generator=g, dtype=torch.float64)
    return B.float().to(device), eo.float().to(device), ev.float().to(device)


def config3_inputs(device, seed: int = 3):
    return pair_inputs(96, 672, 2304, device, seed)


def chain_inputs(nao: int, nocc: int, nvir: int, naux: int, device, seed: int = 4):
    """C4 rules: eri (naux, nao, nao) = 0.02 N(0,1) symmetrised in its last two
    indices as (X + X^T) / sqrt(2) (so entries stay N(0, 0.02^2) off the
    diagonal); C_occ, C_vir the first nocc / next nvir columns of the Q of a
    QR of an N(0,1) (nao x nao) matrix; eps as config 3."""
    g = torch.Generator().manual_seed(seed)
    Mq = torch.randn(nao, nao, generator=g, dtype=torch.float64)
    Q, _ = torch.linalg.qr(Mq)
    C_occ = Q[:, :nocc].contiguous()
    C_vir = Q[:, nocc : nocc + nvir].contiguous()
    eo = -1.5 + 1.2 * torch.rand(nocc, generator=g, dtype=torch.float64)
    ev = 0.1 + 2.9 * torch.rand(nvir, generator=g, dtype=torch.float64)
    gd = torch.Generator(device=device).manual_seed(seed)
    eri = torch.empty((naux, nao, nao), dtype=torch.float32, device=device)
    step = max(1, (1 << 28) // (nao * nao))
    for p0 in range(0, naux, step):
        p1 = min(naux, p0 + step)
        X = 0.02 * torch.randn((p1 - p0, nao, nao), generator=gd, device=device)
        eri[p0:p1] = (X + X.transpose(1, 2)) / math.sqrt(2.0)
    return (
        eri,
        C_occ.float().to(device),
        C_vir.float().to(device),
        eo.float().to(device),
        ev.float().to(device),
    )
