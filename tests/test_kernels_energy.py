"""GPU parity of the fused DF-MP2 pair-energy kernel and the T_flat
reduction kernel (C ABI via trnblas_amd.hip.kernels) against the fp64
closed form of the oracle. Gate: relative 1e-6 (north star)."""

import numpy as np
import pytest
import torch

from oracle import pair_energy as pe

pytestmark = pytest.mark.gpu

MATHS = ["fp32", "bf16x6", "fp16x3"]


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
@pytest.mark.parametrize("math", MATHS)
def test_pair_energy_sym_small(dev, nocc, nvir, naux, math):
    from trnblas_amd.hip import kernels

    B, eo, ev = _inputs(nocc, nvir, naux, nocc * 100 + nvir)
    got = float(kernels.pair_energy_sym(B.to(dev), eo.to(dev), ev.to(dev), math=math))
    want = pe.pair_energy_f64(B, eo, ev)
    assert abs(got - want) <= 1e-6 * abs(want), (got, want)


@pytest.mark.parametrize("math", MATHS)
def test_pair_energy_unaligned_naux(dev, math):
    # naux % 4 != 0 and a strided (non-contiguous) view: scalar-load paths
    from trnblas_amd.hip import kernels

    B, eo, ev = _inputs(4, 100, 63, 9)
    wide = torch.zeros(4, 100, 70)
    wide[:, :, 3:66] = B
    Bv = wide.to(dev)[:, :, 3:66]
    assert not Bv.is_contiguous() and Bv.stride(1) == 70
    got = float(kernels.pair_energy_sym(Bv, eo.to(dev), ev.to(dev), math=math))
    want = pe.pair_energy_f64(B, eo, ev)
    assert abs(got - want) <= 1e-6 * abs(want)


@pytest.mark.parametrize("math", MATHS)
def test_pair_energy_zero_B(dev, math):
    from trnblas_amd.hip import kernels

    B = torch.zeros(3, 50, 40)
    eo = -torch.ones(3)
    ev = torch.ones(50)
    assert float(kernels.pair_energy_sym(B.to(dev), eo.to(dev), ev.to(dev), math=math)) == 0.0


@pytest.mark.parametrize("math", MATHS)
def test_pair_energies_explicit_pairs(dev, math):
    from trnblas_amd.hip import kernels

    B, eo, ev = _inputs(5, 150, 96, 3)
    pairs = [(0, 0), (0, 4), (4, 0), (2, 3), (3, 3), (1, 2)]
    pi = torch.tensor([p[0] for p in pairs])
    pj = torch.tensor([p[1] for p in pairs])
    Bd = B.to(dev)
    got = kernels.pair_energies(Bd, Bd, eo.to(dev), eo.to(dev), ev.to(dev), pi, pj, math=math).cpu()
    want = pe.pair_energies_f64(B, B, eo, eo, ev, pairs)
    assert torch.allclose(got, want, rtol=1e-6, atol=0)
    # e_ij == e_ji (symmetry of the denominator)
    assert abs(got[1] - got[2]) <= 1e-6 * abs(got[1])


@pytest.mark.parametrize("math", MATHS)
def test_pair_energies_two_operands(dev, math):
    # Bi != Bj (the j-batched surface): rows i of Bi against rows j of Bj
    from trnblas_amd.hip import kernels

    Bi, eo, ev = _inputs(3, 120, 70, 11)
    Bj, ej, _ = _inputs(4, 120, 70, 12)
    pairs = [(0, 3), (2, 0), (1, 1), (2, 2)]
    pi = torch.tensor([p[0] for p in pairs])
    pj = torch.tensor([p[1] for p in pairs])
    got = kernels.pair_energies(
        Bi.to(dev), Bj.to(dev), eo.to(dev), ej.to(dev), ev.to(dev), pi, pj, math=math
    ).cpu()
    want = pe.pair_energies_f64(Bi, Bj, eo, ej, ev, pairs)
    assert torch.allclose(got, want, rtol=1e-6, atol=0)


@pytest.mark.parametrize("math,tol", [("fp32", 2.0**-21), ("bf16x6", 2.0**-21), ("fp16x3", 2.0**-19)])
def test_pair_energy_full_significands(dev, math, tol):
    # naux = 1, nvir = 1: T = x y exactly, e = T^2 / D. Operands with all 24
    # significand bits set over a wide exponent range: an fp32-class product
    # is within 2^-22 of x y (bf16x6; a split that lost its lo piece (2^-16)
    # or its mid piece (2^-8) fails). fp16x3 keeps 22 significand bits per
    # operand and drops lo_x lo_y: x y within 3 2^-22, so e within 6 2^-22;
    # without its lo piece it would be off by 2^-11.
    from trnblas_amd.hip import kernels

    g = torch.Generator().manual_seed(5)
    n = 40
    mant = 1.0 + torch.randint(0, 1 << 23, (n,), generator=g).double() / (1 << 23)
    sign = torch.where(torch.rand(n, generator=g) < 0.5, -1.0, 1.0).double()
    x = sign * mant * torch.exp2(torch.randint(-20, 20, (n,), generator=g).double())
    B = x.float().reshape(n, 1, 1)
    eo = -torch.rand(n, generator=g) - 0.5
    ev = torch.tensor([0.7])
    pairs = [(i, (i * 7 + 3) % n) for i in range(n)]
    pi = torch.tensor([p[0] for p in pairs])
    pj = torch.tensor([p[1] for p in pairs])
    Bd = B.to(dev)
    got = kernels.pair_energies(Bd, Bd, eo.to(dev), eo.to(dev), ev.to(dev), pi, pj, math=math).cpu()
    want = pe.pair_energies_f64(B, B, eo, eo, ev, pairs)
    rel = ((got - want).abs() / want.abs()).max().item()
    assert rel <= tol, rel


@pytest.mark.parametrize("math,mean_tol", [("bf16x6", 5e-8), ("fp16x3", 1e-7)])
def test_pair_energy_split_long_sums_unbiased(dev, math, mean_tol):
    # nvir = 1, naux = 2304, pairs (i, i): T = sum_k x_k^2 > 0 and e = T^2 / D.
    # The recovered T must carry no systematic error: summed slice by slice
    # with fp32 adds its mean relative error is ~1e-10 (std ~1e-7); a long
    # sum chained through the MFMA accumulator comes out ~1.5e-6 low.
    # fp16x3 drops lo_x lo_y, which for x = y is positive: x^2 comes out low
    # by lo^2 / x^2, about 2^-22 / 3 times the mean of 1 / m^2 over the
    # significands m in [1, 2), i.e. ~4e-8.
    from trnblas_amd.hip import kernels

    g = torch.Generator().manual_seed(0)
    n, naux = 256, 2304
    B = (0.05 * torch.randn(n, 1, naux, generator=g, dtype=torch.float64)).float()
    eo, ev = -torch.ones(n), torch.tensor([0.5])
    idx = torch.arange(n)
    e = kernels.pair_energies(
        B.to(dev), B.to(dev), eo.to(dev), eo.to(dev), ev.to(dev), idx, idx, math=math
    ).cpu()
    T = (e * -3.0).sqrt()
    Bd = B.double()[:, 0, :]
    T64 = (Bd * Bd).sum(dim=1)
    rel = (T - T64) / T64
    assert abs(float(rel.mean())) <= mean_tol, float(rel.mean())
    assert float(rel.abs().max()) <= 2e-6


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
@pytest.mark.parametrize("math", MATHS)
def test_pair_energy_config3_shape_subset(dev, seed, math):
    # The C3 virtual / aux sizes (672, 2304) at nocc = 6: every tile pair of
    # the production launch shape, against the fp64 closed form.
    from trnblas_amd.hip import kernels

    B, eo, ev = _inputs(6, 672, 2304, seed)
    got = float(kernels.pair_energy_sym(B.to(dev), eo.to(dev), ev.to(dev), math=math))
    want = pe.pair_energy_f64(B, eo, ev)
    assert abs(got - want) <= 1e-6 * abs(want), (got, want)


@pytest.mark.parametrize("math", ["bf16x6", "fp16x3"])
@pytest.mark.parametrize("nocc,nvir,naux", [(5, 97, 130), (8, 200, 64), (1, 33, 40)])
def test_pair_energy_split_implicit_walk_per_pair(dev, nocc, nvir, naux, math):
    # the implicit walk runs two pairs (i, j), (i, j + 1) per workgroup; its
    # per-pair energies (out_pairs, row-major i <= j) must match the
    # explicit-pair kernel's, pair by pair (odd rows leave a single pair)
    from trnblas_amd.hip import kernels

    B, eo, ev = _inputs(nocc, nvir, naux, seed=nocc + nvir)
    B, eo, ev = B.to(dev), eo.to(dev), ev.to(dev)
    npairs = nocc * (nocc + 1) // 2
    got = torch.empty(npairs, dtype=torch.float64, device=dev)
    tot = torch.empty((), dtype=torch.float64, device=dev)
    kernels._pe_launch(
        math, dev, nvir, naux, B, nocc, B.stride(0), B, 0, B.stride(0), B.stride(1),
        eo, eo, ev, nocc, npairs, None, None, got, tot,
    )  # fmt: skip
    ii, jj = np.triu_indices(nocc)
    want = kernels.pair_energies(B, B, eo, eo, ev, torch.from_numpy(ii), torch.from_numpy(jj), math=math)
    torch.cuda.synchronize()
    scale = float(want.abs().max()) + 1e-300
    assert float((got - want).abs().max()) <= 1e-12 * scale
    w = torch.where(torch.from_numpy(ii == jj).to(dev), 1.0, 2.0).double()
    assert abs(float(tot) - float((w * want).sum())) <= 1e-12 * abs(float(tot))


@pytest.mark.parametrize("math", MATHS)
def test_pair_energy_wide_dynamic_range(dev, math):
    # Rows whose scales span e^-8 .. e^8 and elements spanning e^-6 .. e^6
    # within a row, plus an all-zero row and a row of one nonzero element:
    # fp16x3's per-row power-of-two scaling must keep every row in fp16's
    # range (small elements fall into its subnormals), bf16x6 has fp32's
    # exponent range. Relative 1e-6 against the fp64 closed form.
    from trnblas_amd.hip import kernels

    g = torch.Generator().manual_seed(11)
    nocc, nvir, naux = 4, 150, 200
    row = torch.exp(4.0 * torch.randn(nocc, nvir, 1, generator=g, dtype=torch.float64))
    elem = torch.exp(2.0 * torch.randn(nocc, nvir, naux, generator=g, dtype=torch.float64))
    B = 0.05 * row * elem * torch.randn(nocc, nvir, naux, generator=g, dtype=torch.float64)
    B[1, 7] = 0.0
    B[2, 9] = 0.0
    B[2, 9, 17] = 3.0
    B = B.float()
    eo = -0.3 - 1.2 * torch.rand(nocc, generator=g, dtype=torch.float64)
    ev = 0.1 + 2.9 * torch.rand(nvir, generator=g, dtype=torch.float64)
    got = float(kernels.pair_energy_sym(B.to(dev), eo.float().to(dev), ev.float().to(dev), math=math))
    want = pe.pair_energy_f64(B, eo.float(), ev.float())
    assert abs(got - want) <= 1e-6 * abs(want), (got, want)


@pytest.mark.parametrize("math,tol", [("fp32", 1e-6), ("bf16x6", 1e-6), ("fp16x3", 1e-6)])
def test_pair_energy_wide_range_rows(dev, math, tol):
    # rows whose entries spread over 2^-16 .. 2^16 of each other: fp16x3 scales
    # each row so its largest entry sits at 2^14, so entries 2^-28 below it
    # are fp16 subnormals and keep an absolute error (<= 2^-39 of the row
    # maximum) instead of a relative one. The energy is a sum of products
    # dominated by the large entries; the gate is the same rel 1e-6 against
    # fp64, and the measured error of each arithmetic is printed.
    from trnblas_amd.hip import kernels

    g = torch.Generator().manual_seed(17)
    nocc, nvir, naux = 6, 130, 200
    B = torch.randn(nocc, nvir, naux, generator=g, dtype=torch.float64)
    B = B * torch.exp2(torch.randint(-16, 17, (nocc, nvir, naux), generator=g).double()) * 0.05
    B = B.float()
    eo = -1.5 + 1.2 * torch.rand(nocc, generator=g)
    ev = 0.1 + 2.9 * torch.rand(nvir, generator=g)
    got = float(kernels.pair_energy_sym(B.to(dev), eo.to(dev), ev.to(dev), math=math))
    want = pe.pair_energy_f64(B, eo, ev)
    rel = abs(got - want) / abs(want)
    print(f"wide-range rows, {math}: rel {rel:.2e}", flush=True)
    assert rel <= tol, rel
