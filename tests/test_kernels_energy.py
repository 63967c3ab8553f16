"""GPU parity of the fused DF-MP2 pair-energy kernel and the T_flat
reduction kernel (C ABI via trnblas_amd.hip.kernels) against the fp64
closed form of the oracle. Gate: relative 1e-6 (north star)."""

import pytest
import torch

from oracle import pair_energy as pe

pytestmark = pytest.mark.gpu


def _inputs(nocc, nvir, naux, seed):
    g = torch.Generator().manual_seed(seed)
    B = torch.randn(nocc, nvir, naux, generator=g, dtype=torch.float64) * 0.05
    eo = -0.3 - 1.2 * torch.rand(nocc, generator=g, dtype=torch.float64)
    ev = 0.1 + 2.9 * torch.rand(nvir, generator=g, dtype=torch.float64)
    return B.float(), eo.float(), ev.float()


@pytest.mark.parametrize(
    "nocc,nvir,naux",
    [(1, 1, 1), (3, 96, 128), (5, 97, 130), (4, 200, 77), (7, 130, 300), (2, 300, 5), (6, 33, 16)],
)
def test_pair_energy_sym_small(dev, nocc, nvir, naux):
    from trnblas_amd.hip import kernels

    B, eo, ev = _inputs(nocc, nvir, naux, nocc * 100 + nvir)
    got = float(kernels.pair_energy_sym(B.to(dev), eo.to(dev), ev.to(dev)))
    want = pe.pair_energy_f64(B, eo, ev)
    assert abs(got - want) <= 1e-6 * abs(want), (got, want)


def test_pair_energy_unaligned_naux(dev):
    # naux % 4 != 0 and a non-contiguous view: scalar-load path
    from trnblas_amd.hip import kernels

    B, eo, ev = _inputs(4, 100, 63, 9)
    Bv = B.to(dev)
    got = float(kernels.pair_energy_sym(Bv, eo.to(dev), ev.to(dev)))
    want = pe.pair_energy_f64(B, eo, ev)
    assert abs(got - want) <= 1e-6 * abs(want)


def test_pair_energy_zero_B(dev):
    from trnblas_amd.hip import kernels

    B = torch.zeros(3, 50, 40)
    eo = -torch.ones(3)
    ev = torch.ones(50)
    assert float(kernels.pair_energy_sym(B.to(dev), eo.to(dev), ev.to(dev))) == 0.0


def test_pair_energies_explicit_pairs(dev):
    from trnblas_amd.hip import kernels

    B, eo, ev = _inputs(5, 150, 96, 3)
    pairs = [(0, 0), (0, 4), (4, 0), (2, 3), (3, 3), (1, 2)]
    pi = torch.tensor([p[0] for p in pairs])
    pj = torch.tensor([p[1] for p in pairs])
    Bd = B.to(dev)
    got = kernels.pair_energies(Bd, Bd, eo.to(dev), eo.to(dev), ev.to(dev), pi, pj).cpu()
    want = pe.pair_energies_f64(B, B, eo, eo, ev, pairs)
    assert torch.allclose(got, want, rtol=1e-6, atol=0)
    # e_ij == e_ji (symmetry of the denominator)
    assert abs(got[1] - got[2]) <= 1e-6 * abs(got[1])


def test_mp2_energy_kernel(dev):
    from trnblas_amd.hip import kernels

    B, eo, ev = _inputs(4, 70, 50, 5)
    nocc, nvir, naux = B.shape
    flat = B.reshape(nocc * nvir, naux)
    T_flat = (flat[: 2 * nvir].double() @ flat.double().T).float()  # ic = 2
    got = kernels.mp2_energy_pairs(T_flat.to(dev), eo[:2].to(dev), eo.to(dev), ev.to(dev))
    want = pe.mp2_energy_cpu(T_flat.double(), eo[:2].double(), eo.double(), ev.double())
    assert abs(float(got.sum()) - float(want)) <= 1e-9 * abs(float(want))


@pytest.mark.parametrize("seed", [0])
def test_pair_energy_config3_shape_subset(dev, seed):
    # The C3 virtual / aux sizes (672, 2304) at nocc = 6: every tile pair of
    # the production launch shape, against the fp64 closed form.
    from trnblas_amd.hip import kernels

    B, eo, ev = _inputs(6, 672, 2304, seed)
    got = float(kernels.pair_energy_sym(B.to(dev), eo.to(dev), ev.to(dev)))
    want = pe.pair_energy_f64(B, eo, ev)
    assert abs(got - want) <= 1e-6 * abs(want), (got, want)
