"""Pins the DF-MP2 chain oracle (oracle/df_mp2.py) by properties that do
not restate its formula: auxiliary-basis rotation invariance, independence
of the factor of J^-1, and the J = I / identity-orbital composition."""

import numpy as np
import torch

from oracle import df_mp2 as od
from oracle import metric as om
from oracle import pair_energy as pe


def _inputs(nbasis=12, nocc=3, naux=10, seed=0):
    rng = np.random.default_rng(seed)
    C_occ = 0.3 * rng.standard_normal((nbasis, nocc))
    C_vir = 0.3 * rng.standard_normal((nbasis, nbasis - nocc))
    eri = 0.1 * rng.standard_normal((nbasis, nbasis, naux))
    J = om.spd(naux, seed=seed + 1)
    eo = -0.5 - np.sort(rng.random(nocc))
    ev = 0.1 + np.sort(rng.random(nbasis - nocc))
    return C_occ, C_vir, eri, J, eo, ev


def test_aux_rotation_invariance():
    C_occ, C_vir, eri, J, eo, ev = _inputs()
    Q, _ = np.linalg.qr(np.random.default_rng(5).standard_normal((J.shape[0],) * 2))
    e0 = od.df_mp2_energy_ref(C_occ, C_vir, eri, J, eo, ev)
    e1 = od.df_mp2_energy_ref(C_occ, C_vir, eri @ Q, Q.T @ J @ Q, eo, ev)
    assert abs(e1 - e0) <= 1e-12 * abs(e0)


def test_planted_transposed_factor_breaks_rotation_invariance():
    # the mistake the rotation check is there to catch: B = (ia|P) X^T
    C_occ, C_vir, eri, J, eo, ev = _inputs(seed=1)
    Q, _ = np.linalg.qr(np.random.default_rng(6).standard_normal((J.shape[0],) * 2))
    Xt = om.metric_inv_half_ref(J).T
    Jr = Q.T @ J @ Q
    e0 = od.df_mp2_energy_ref(C_occ, C_vir, eri, J, eo, ev, factor=Xt)
    e1 = od.df_mp2_energy_ref(C_occ, C_vir, eri @ Q, Jr, eo, ev, factor=om.metric_inv_half_ref(Jr).T)
    assert abs(e1 - e0) > 1e-6 * abs(e0)


def test_factor_independence():
    C_occ, C_vir, eri, J, eo, ev = _inputs(seed=2)
    e0 = od.df_mp2_energy_ref(C_occ, C_vir, eri, J, eo, ev)
    e1 = od.df_mp2_energy_ref(C_occ, C_vir, eri, J, eo, ev, factor=od.inv_sqrt_sym(J))
    assert abs(e1 - e0) <= 1e-12 * abs(e0)
    S = od.inv_sqrt_sym(J)
    assert np.allclose(S @ S @ J, np.eye(J.shape[0]), atol=1e-12)


def test_identity_metric_and_orbitals_reduce_to_the_pair_energy():
    # J = I, C_occ = the first nocc columns of I, C_vir the rest: B[i, a, P]
    # = eri[i, nocc + a, P], and the chain's energy is that block's pair energy
    nbasis, nocc, naux = 10, 3, 7
    _, _, eri, _, eo, ev = _inputs(nbasis, nocc, naux, seed=3)
    I = np.eye(nbasis)
    e = od.df_mp2_energy_ref(I[:, :nocc], I[:, nocc:], eri, np.eye(naux), eo, ev)
    B = torch.from_numpy(eri[:nocc, nocc:, :].copy())
    want = pe.pair_energy_f64(B, torch.from_numpy(eo), torch.from_numpy(ev))
    assert abs(e - want) <= 1e-13 * abs(want)
