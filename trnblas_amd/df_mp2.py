"""The DF-MP2 energy step (and the config-4 chain) on trnblas_amd.

The MI355X counterpart of the energy step of examples/df_mp2.py:
* `energy_reduction` — the example's default path (df_mp2.py:51-99):
  chunked `gemm(B_chunk, B_flat, transB=True)` + torch reduction;
* `energy_reduction_batched_pair` — its `--batched-pair-energy` path
  (df_mp2.py:131-144): one fused HIP launch for every pair;
* `df_mp2_energy` — the example's whole calculation (df_mp2.py:147-233):
  metric factor, half-transforms, metric contraction, energy, with its four
  energy paths (`energy_reduction` with / without `use_fused`,
  `energy_reduction_fused_gemm`, `energy_reduction_batched_pair`), and its
  `flops` / `make_inputs` helpers;
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


def energy_reduction(
    B, eps_occ, eps_vir, *, mem_budget_bytes: int = 1_500_000_000, use_fused: bool = False
) -> float:
    """E = sum_{ijab} T_ijab (2 T_ijab - T_ijba) / D_ijab by chunked GEMM
    (one `gemm(..., transB=True)` per i-chunk, B_flat^T read in place) and a
    torch reduction, or with `use_fused` the `mp2_energy` HIP reduction of
    each T chunk (examples/df_mp2.py:51-99)."""
    nocc, nvir, naux = B.shape
    i_block = max(1, min(nocc, int(mem_budget_bytes // (4 * nvir * nocc * nvir))))
    flat = B.reshape(nocc * nvir, naux)
    if not use_fused:
        eo2 = eps_occ.view(nocc, 1, 1, 1) + eps_occ.view(1, nocc, 1, 1)
        ev2 = eps_vir.view(1, 1, nvir, 1) + eps_vir.view(1, 1, 1, nvir)
    e = torch.zeros((), dtype=B.dtype, device=B.device)
    for i0 in range(0, nocc, i_block):
        i1 = min(i0 + i_block, nocc)
        T_flat = level3.gemm(1.0, flat[i0 * nvir : i1 * nvir], flat, transB=True)
        if use_fused:
            e = e + _d.nki_mp2_energy(T_flat, eps_occ[i0:i1], eps_occ, eps_vir)
            continue
        T = T_flat.reshape(i1 - i0, nvir, nocc, nvir).permute(0, 2, 1, 3)
        e = e + (T * (2.0 * T - T.transpose(-2, -1)) / (eo2[i0:i1] - ev2)).sum()
    return float(e)


def energy_reduction_fused_gemm(B, eps_occ, eps_vir) -> float:
    """The per-pair fused GEMM + energy loop over all nocc^2 ordered pairs
    (examples/df_mp2.py:102-128), one fused HIP launch per pair."""
    nocc = B.shape[0]
    e = torch.zeros((), dtype=B.dtype, device=B.device)
    for i in range(nocc):
        for j in range(nocc):
            e = e + _d.nki_fused_gemm_energy(B[i], B[j], float(eps_occ[i]), float(eps_occ[j]), eps_vir)
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


def df_mp2_energy(
    C_occ: torch.Tensor,
    C_vir: torch.Tensor,
    eri_3c: torch.Tensor,
    J_metric: torch.Tensor,
    eps_occ: torch.Tensor,
    eps_vir: torch.Tensor,
    timings: dict | None = None,
    use_fused: bool = False,
    use_fused_gemm: bool = False,
    use_batched_pair: bool = False,
) -> float:
    """DF-MP2 correlation energy (examples/df_mp2.py:147-233), the
    reference's layout and steps: eri_3c is (nbasis, nbasis, naux), C_occ
    (nbasis, nocc), C_vir (nbasis, nvir), J_metric (naux, naux).

    1. X = metric_inv_half(J) (X = L^-T, J = L L^T; fp64 on the device);
    2a. (i nu|P) = C_occ^T (mu nu|P): one GEMM on the (nbasis, nbasis naux)
        view of eri (transA, read in place);
    2b. (ia|P) = C_vir^T (i nu|P)_i: one batched GEMM whose C_vir^T operand
        is a stride-0 broadcast (no per-batch copies);
    3. B_i = (ia|P)_i X: one batched GEMM, X broadcast the same way;
    4. the energy, by `use_batched_pair` (the fused pair-energy kernel, one
       launch), `use_fused_gemm` (one fused launch per ordered pair),
       `use_fused` (chunked GEMM + the HIP mp2_energy reduction) or the
       default chunked GEMM + torch reduction.
    `timings` receives seconds per step (chol, half, metric, energy)."""
    import time

    nbasis, nocc = C_occ.shape
    nvir = C_vir.shape[1]
    naux = J_metric.shape[0]
    dev = C_occ.device

    def sync():
        if timings is not None and dev.type == "cuda":
            torch.cuda.synchronize(dev)

    t0 = time.perf_counter()
    X = level3.metric_inv_half(J_metric)
    sync()
    t_chol = time.perf_counter() - t0

    t0 = time.perf_counter()
    eri_flat = eri_3c.reshape(nbasis, nbasis * naux)
    iv_P = level3.gemm(1.0, C_occ, eri_flat, transA=True).reshape(nocc, nbasis, naux)
    ia_P = level3.batched_gemm(1.0, C_vir.mT.unsqueeze(0).expand(nocc, nvir, nbasis), iv_P)
    sync()
    t_half = time.perf_counter() - t0

    t0 = time.perf_counter()
    B = level3.batched_gemm(1.0, ia_P, X.to(ia_P.dtype).unsqueeze(0).expand(nocc, naux, naux))
    sync()
    t_metric = time.perf_counter() - t0

    t0 = time.perf_counter()
    if use_batched_pair:
        e = energy_reduction_batched_pair(B, eps_occ, eps_vir)
    elif use_fused_gemm:
        e = energy_reduction_fused_gemm(B, eps_occ, eps_vir)
    else:
        e = energy_reduction(B, eps_occ, eps_vir, use_fused=use_fused)
    t_energy = time.perf_counter() - t0
    if timings is not None:
        timings.update(chol=t_chol, half=t_half, metric=t_metric, energy=t_energy)
    return float(e)


def flops(nbasis: int, nocc: int, naux: int) -> int:
    """Approximate flops of one df_mp2_energy (examples/df_mp2.py:236-242):
    steps 2a, 2b, 3 and the ordered-pair energy GEMMs."""
    nvir = nbasis - nocc
    return (
        2 * nbasis * nbasis * nocc * naux
        + 2 * nocc * nvir * nbasis * naux
        + 2 * nocc * nvir * naux * naux
        + 2 * nocc * nocc * nvir * nvir * naux
    )


def make_inputs(nbasis: int, nocc: int, naux: int, seed: int = 42, device: str = "cpu"):
    """The example's synthetic inputs (examples/df_mp2.py:245-266): the same
    draws in the same order from torch's global generator on the host, then
    moved to `device`. Returns (C_occ, C_vir, eri_3c, J_metric, eps_occ,
    eps_vir)."""
    torch.manual_seed(seed)
    C_occ = torch.randn(nbasis, nocc) * 0.1
    C_vir = torch.randn(nbasis, nbasis - nocc) * 0.1
    eri_3c = torch.randn(nbasis, nbasis, naux) * 0.01
    J_raw = torch.randn(naux, naux) * 0.01
    J_metric = J_raw @ J_raw.T + naux * torch.eye(naux)
    eps_occ = -torch.sort(torch.rand(nocc))[0] - 0.5
    eps_vir = torch.sort(torch.rand(nbasis - nocc))[0] + 0.1
    return tuple(t.to(device) for t in (C_occ, C_vir, eri_3c, J_metric, eps_occ, eps_vir))


# The example's benchmark shapes (examples/df_mp2.py:269-273), as
# (nbasis, nocc, naux); "large" has nvir 672, the C3 pair-energy shape.
BENCH_SHAPES = {
    "small": (128, 16, 384),
    "medium": (512, 64, 1536),
    "large": (768, 96, 2304),
}


def bench(shape_name: str, device: str = "cpu", use_fused: bool = False, use_fused_gemm: bool = False,
          use_batched_pair: bool = False, passes: str = "both", verbose: bool = True) -> list:
    """Cold and / or warm timing of one `df_mp2_energy` at a bench shape (the
    example's `bench`, examples/df_mp2.py:276-333): per-step seconds, total,
    approximate TFLOP/s and the energy E, one dict per pass (also printed).
    On the GPU the cold pass includes loading the kernels; there is no
    per-shape compile, so the two passes differ by little."""
    import time

    nbasis, nocc, naux = BENCH_SHAPES[shape_name]
    nvir = nbasis - nocc
    fl = flops(nbasis, nocc, naux)
    inputs = make_inputs(nbasis, nocc, naux, device=device)
    mode = ("batched-pair" if use_batched_pair else "fused-gemm" if use_fused_gemm
            else "fused" if use_fused else "torch")  # fmt: skip
    if verbose:
        print(f"[shape={shape_name} nbasis={nbasis} nocc={nocc} nvir={nvir} naux={naux}]")
        print(f"  approx flops: {fl / 1e9:.1f} G  backend: {_d.get_backend()}  device: {device}  "
              f"energy_mode: {mode}")  # fmt: skip
    out = []
    for label in {"cold": ["cold"], "warm": ["warm"], "both": ["cold", "warm"]}[passes]:
        t: dict = {}
        t0 = time.perf_counter()
        e = df_mp2_energy(*inputs, timings=t, use_fused=use_fused, use_fused_gemm=use_fused_gemm,
                          use_batched_pair=use_batched_pair)  # fmt: skip
        if torch.device(device).type == "cuda":
            torch.cuda.synchronize()
        total = time.perf_counter() - t0
        row = dict(pass_=label, shape=shape_name, mode=mode, total=total, tflops=fl / total / 1e12,
                   E=e, **t)  # fmt: skip
        out.append(row)
        if verbose:
            print(f"  {label}: chol {t['chol']:.3f}s  half {t['half']:.3f}s  metric {t['metric']:.3f}s  "
                  f"energy {t['energy']:.3f}s  total {total:.3f}s  ~{row['tflops']:.2f} TFLOPS  E={e:.6e}")
    return out


def main(argv=None) -> None:
    """The example's command line (examples/df_mp2.py:336-428):
    python -m trnblas_amd.df_mp2 [--bench [--shape S]] [--demo] [--nbasis N
    --nocc O --naux P] [--device cuda] [--fused-energy | --fused-gemm-energy
    | --batched-pair-energy] [--passes cold|warm|both]."""
    import argparse
    import time

    ap = argparse.ArgumentParser(description="DF-MP2 using trnblas_amd")
    ap.add_argument("--demo", action="store_true", help="small demo (water-like)")
    ap.add_argument("--bench", action="store_true", help="cold / warm timing of the bench shapes")
    ap.add_argument("--shape", choices=list(BENCH_SHAPES), help="restrict --bench to one shape")
    ap.add_argument("--nbasis", type=int, default=24)
    ap.add_argument("--nocc", type=int, default=5)
    ap.add_argument("--naux", type=int, default=None)
    ap.add_argument("--device", default="cpu", help="torch device of the inputs (cpu, cuda, cuda:0 ...)")
    ap.add_argument("--fused-energy", action="store_true", help="chunked GEMM + the HIP mp2_energy reduction")
    ap.add_argument("--fused-gemm-energy", action="store_true", help="one fused launch per ordered pair")
    ap.add_argument("--batched-pair-energy", action="store_true", help="the fused pair energy, one launch")
    ap.add_argument("--passes", choices=["cold", "warm", "both"], default="both")
    a = ap.parse_args(argv)
    kw = dict(use_fused=a.fused_energy, use_fused_gemm=a.fused_gemm_energy,
              use_batched_pair=a.batched_pair_energy)  # fmt: skip
    if a.bench:
        for shape in [a.shape] if a.shape else list(BENCH_SHAPES):
            bench(shape, device=a.device, passes=a.passes, **kw)
        return
    if a.demo:
        a.nbasis, a.nocc = 24, 5
    nbasis, nocc = a.nbasis, a.nocc
    naux = a.naux or 3 * nbasis
    inputs = make_inputs(nbasis, nocc, naux, device=a.device)
    print(f"DF-MP2: nbasis {nbasis}, nocc {nocc}, nvir {nbasis - nocc}, naux {naux}, "
          f"backend {_d.get_backend()}")  # fmt: skip
    t: dict = {}
    t0 = time.perf_counter()
    e = df_mp2_energy(*inputs, timings=t, **kw)
    total = time.perf_counter() - t0
    for k, v in t.items():
        print(f"  {k:15s}: {v:.3f}s")
    print(f"\n  E_MP2 = {e:.10f} (synthetic data)\n  Total: {total:.3f}s")


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


def config5_inputs(device, n: int = 8192, seed: int = 5):
    """C5 rules: A, B (n x n) fp64, each entry U(-1, 1) 2^round(N(0, 4^2)),
    drawn on the host CPU from torch.Generator().manual_seed(seed) in the
    order A's uniforms, A's exponents, B's uniforms, B's exponents, then
    copied to `device` (the same values on every machine with this torch's
    CPU generator)."""
    g = torch.Generator().manual_seed(seed)

    def draw():
        u = torch.rand(n, n, generator=g, dtype=torch.float64) * 2 - 1
        e = torch.round(4.0 * torch.randn(n, n, generator=g, dtype=torch.float64))
        return (u * torch.exp2(e)).to(device)

    A = draw()
    return A, draw()


def chain_inputs(nao: int, nocc: int, nvir: int, naux: int, device, seed: int = 4):
    """C4 rules: eri (naux, nao, nao) = 0.02 N(0,1) symmetrised in its last two
    indices as (X + X^T) / sqrt(2) (so entries stay N(0, 0.02^2) off the
    diagonal); C_occ, C_vir the first nocc / next nvir columns of the Q of a
    QR of an N(0,1) (nao x nao) matrix; eps as config 3.

    Everything is drawn on the host CPU from torch.Generator().manual_seed(
    seed), in that order: the QR matrix and eps in fp64, then X in fp32 in
    fixed chunks of 2^26 values (whole P-slices), each chunk copied to
    `device` and symmetrised there. X is drawn in fp32 rather than fp64
    because 4.3e9 fp64 normals take about a minute on the GPU box's host
    (fp32: ~12 s)."""
    g = torch.Generator().manual_seed(seed)
    Mq = torch.randn(nao, nao, generator=g, dtype=torch.float64)
    Q, _ = torch.linalg.qr(Mq)
    C_occ = Q[:, :nocc].contiguous()
    C_vir = Q[:, nocc : nocc + nvir].contiguous()
    eo = -1.5 + 1.2 * torch.rand(nocc, generator=g, dtype=torch.float64)
    ev = 0.1 + 2.9 * torch.rand(nvir, generator=g, dtype=torch.float64)
    eri = torch.empty((naux, nao, nao), dtype=torch.float32, device=device)
    step = max(1, (1 << 26) // (nao * nao))
    scale = 0.02 / math.sqrt(2.0)
    for p0 in range(0, naux, step):
        p1 = min(naux, p0 + step)
        X = torch.randn((p1 - p0, nao, nao), generator=g, dtype=torch.float32).to(device)
        eri[p0:p1] = (X + X.transpose(1, 2)) * scale
        del X
    return (
        eri,
        C_occ.float().to(device),
        C_vir.float().to(device),
        eo.float().to(device),
        ev.float().to(device),
    )


if __name__ == "__main__":
    main()
