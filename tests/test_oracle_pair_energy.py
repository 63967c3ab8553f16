"""Pins of the pair-energy oracle (oracle/pair_energy.py), CPU only."""

import pytest
import torch

from oracle import pair_energy as pe


def _inp(nocc, nvir, naux, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    B = 0.05 * torch.randn(nocc, nvir, naux, generator=g, dtype=torch.float64)
    eo = -1.5 + 1.2 * torch.rand(nocc, generator=g, dtype=torch.float64)
    ev = 0.1 + 2.9 * torch.rand(nvir, generator=g, dtype=torch.float64)
    return B.to(dtype), eo.to(dtype), ev.to(dtype)


def _brute(B, eo, ev):
    tot = 0.0
    n, v, _ = B.shape
    for i in range(n):
        for j in range(n):
            for a in range(v):
                for b in range(v):
                    tab = float(B[i, a] @ B[j, b])
                    tba = float(B[i, b] @ B[j, a])
                    tot += tab * (2 * tab - tba) / float(eo[i] + eo[j] - ev[a] - ev[b])
    return tot


def test_forms_agree_with_brute_force():
    B, eo, ev = _inp(3, 5, 4, 1)
    ref = _brute(B, eo, ev)
    for got in (
        pe.pair_energy_f64(B, eo, ev),
        pe.pair_energy_f64_full(B, eo, ev),
        float(pe.batched_pair_cpu(B, eo, ev)),
        float(pe.chunked_pair_cpu(B, eo, ev)),
        pe.energy_reduction_cpu(B, eo, ev),
    ):
        assert abs(got - ref) <= 1e-12 * abs(ref)


def test_symmetric_walk_equals_full_loop():
    B, eo, ev = _inp(7, 30, 20, 2)
    a, b = pe.pair_energy_f64(B, eo, ev), pe.pair_energy_f64_full(B, eo, ev)
    assert abs(a - b) <= 1e-12 * abs(b)


def test_zero_B_and_rank_one_closed_form():
    B, eo, ev = _inp(3, 6, 5, 3)
    assert pe.pair_energy_f64(torch.zeros_like(B), eo, ev) == 0.0
    # rank one: B[i, a, :] = x_i y_a u (|u| = 1) -> T_ab = x_i x_j y_a y_b = T_ba,
    # E = sum_ij sum_ab (x_i x_j y_a y_b)^2 / D
    x = torch.tensor([0.3, -0.7, 0.5], dtype=torch.float64)
    y = torch.linspace(-1, 1, 6, dtype=torch.float64)
    u = torch.zeros(5, dtype=torch.float64)
    u[2] = 1.0
    Br = x[:, None, None] * y[None, :, None] * u
    want = sum(
        float(((x[i] * x[j] * y[:, None] * y[None, :]) ** 2 / (eo[i] + eo[j] - ev[:, None] - ev[None, :])).sum())
        for i in range(3)
        for j in range(3)
    )
    assert abs(pe.pair_energy_f64(Br, eo, ev) - want) <= 1e-13 * abs(want)


def test_virtual_permutation_invariance_and_pair_symmetry():
    B, eo, ev = _inp(4, 12, 7, 4)
    p = torch.randperm(12, generator=torch.Generator().manual_seed(1))
    a, b = pe.pair_energy_f64(B, eo, ev), pe.pair_energy_f64(B[:, p], eo, ev[p])
    assert abs(a - b) <= 1e-13 * abs(a)
    e = pe.pair_energies_f64(B, B, eo, eo, ev, [(0, 3), (3, 0)])
    assert abs(e[0] - e[1]) <= 1e-14 * abs(e[0])


def test_planted_missing_exchange_term_is_caught():
    # dropping the -T_ba exchange term changes the energy: the checks see it
    B, eo, ev = _inp(3, 8, 6, 5)
    ref = pe.pair_energy_f64_full(B, eo, ev)
    Bd, eod, evd = B.double(), eo.double(), ev.double()
    wrong = 0.0
    for i in range(3):
        for j in range(3):
            T = Bd[i] @ Bd[j].T
            wrong += float((T * 2.0 * T / (eod[i] + eod[j] - evd[:, None] - evd[None, :])).sum())
    assert abs(wrong - ref) > 1e-3 * abs(ref)


@pytest.mark.parametrize(
    "nocc,weights",
    [(1, [1.0, 0.0]), (2, [1.0, 1.0]), (3, [1.0, 2.0]), (4, [1.0, 2.0, 1.0, 0.0]), (5, [1.0, 2.0, 2.0, 0.0])],
)
def test_pair_sym_window_weights(nocc, weights):
    # each unordered pair once: weights sum to nocc^2 / nocc (known answers)
    dims = pe.pair_sym_dims(nocc, 100, 200)
    assert dims["weights"] == weights
    assert sum(dims["weights"]) * nocc == nocc * nocc
    assert dims["nd_pad"] % 2 == 0


def test_mp2_energy_cpu_matches_closed_form():
    B, eo, ev = _inp(4, 9, 6, 6)
    nocc, nvir, naux = B.shape
    flat = B.reshape(nocc * nvir, naux)
    total = 0.0
    for i0 in range(0, nocc, 2):
        T_flat = flat[i0 * nvir : (i0 + 2) * nvir] @ flat.T
        total += float(pe.mp2_energy_cpu(T_flat, eo[i0 : i0 + 2], eo, ev))
    ref = pe.pair_energy_f64_full(B, eo, ev)
    assert abs(total - ref) <= 1e-12 * abs(ref)
