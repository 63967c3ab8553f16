"""Config 4 at its real size: the DF-MP2 chain (nao 1024, nocc 256, nvir 768,
naux 4096; seed 4) — two half-transform batched GEMMs into B (256 x 768 x
4096 fp32, 3.2 GB, read by the fused energy kernel in place) and the fused
pair energy — against an fp64 evaluation of the same chain on the device
(fp64 half-transforms, then the fp64 i <= j walk). Gate: relative 1e-6
(north star). The chain follows examples/df_mp2.py:185-224 with the P-major
3-center layout of the configuration."""

import time

import pytest
import torch

from trnblas_amd import df_mp2

pytestmark = pytest.mark.gpu

NAO, NOCC, NVIR, NAUX = 1024, 256, 768, 4096


def _half_transform_f64(eri, Co, Cv, chunk=256):
    """B[i, a, P] = sum_{mu nu} Co[mu, i] Cv[nu, a] eri[P, mu, nu] in fp64,
    a chunk of P at a time (the fp64 copy of the whole eri would be 34 GB)."""
    naux = eri.shape[0]
    Cod, Cvd = Co.double(), Cv.double()
    B = torch.empty((Co.shape[1], Cv.shape[1], naux), dtype=torch.float64, device=eri.device)
    for p0 in range(0, naux, chunk):
        E = eri[p0 : p0 + chunk].double()  # (c, nao, nao)
        T1 = torch.matmul(Cod.T.contiguous(), E)  # (c, nocc, nao)
        B[:, :, p0 : p0 + chunk] = torch.matmul(T1, Cvd).permute(1, 2, 0)  # (nocc, nvir, c)
        del E, T1
    return B


def _pair_energy_f64(B64, eo, ev):
    """sum_{i <= j} w_ij sum_ab T (2T - T^T) / D with T = B_i B_j^T, w = 1 / 2,
    all in fp64 (the reference's energy formula, dispatch.py:2514-2533)."""
    eod, evd = eo.double(), ev.double()
    nocc = B64.shape[0]
    tot = torch.zeros((), dtype=torch.float64, device=B64.device)
    for i in range(nocc):
        T = torch.matmul(B64[i].unsqueeze(0), B64[i:].transpose(1, 2))
        D = eod[i] + eod[i:, None, None] - evd[None, :, None] - evd[None, None, :]
        e = (T * (2.0 * T - T.transpose(1, 2)) / D).sum(dim=(1, 2))
        w = torch.full_like(e, 2.0)
        w[0] = 1.0
        tot += (w * e).sum()
        del T, D, e
    return float(tot)


def test_config4_chain_full_size(dev):
    t0 = time.perf_counter()
    eri, Co, Cv, eo, ev = df_mp2.chain_inputs(NAO, NOCC, NVIR, NAUX, dev, seed=4)
    timings = {}
    e = df_mp2.df_mp2_chain_energy(eri, Co, Cv, eo, ev, timings=timings)
    B = df_mp2.half_transform(eri, Co, Cv)
    assert B.shape == (NOCC, NVIR, NAUX) and B.stride(2) == 1
    B64 = _half_transform_f64(eri, Co, Cv)
    del eri
    # the fp32 half-transforms: componentwise against fp64 (|C| sums bound them)
    err_b = float((B.double() - B64).abs().max() / B64.abs().max())
    del B
    torch.cuda.empty_cache()
    want = _pair_energy_f64(B64, eo, ev)
    rel = abs(e - want) / abs(want)
    print(f"config4: E {e!r} fp64 {want!r} rel {rel:.3e} B err {err_b:.2e} "
          f"half {timings['half']*1e3:.1f} ms energy {timings['energy']*1e3:.1f} ms "
          f"test {time.perf_counter() - t0:.1f} s", flush=True)
    assert err_b <= 1e-5
    assert rel <= 1e-6, (e, want)
    del B64
    torch.cuda.empty_cache()
