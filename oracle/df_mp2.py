"""Oracle: the DF-MP2 calculation of trnblas's example, restated.

Test infrastructure only (see oracle/__init__.py).

* `df_mp2_energy_ref`  examples/df_mp2.py:147-233 in float64 numpy:
                       X = metric_inv_half_ref(J) (X = L^-T, J = L L^T),
                       (i nu|P) = sum_mu C_occ[mu, i] eri[mu, nu, P],
                       (ia|P) = sum_nu C_vir[nu, a] (i nu|P),
                       B_i = (ia|P)_i X, and the energy of B by
                       pair_energy.pair_energy_f64 (both oracles pinned on
                       their own); `factor` replaces L^-T by any X with
                       X X^T = J^-1.
* `inv_sqrt_sym`       the symmetric J^-1/2 (eigendecomposition), a second
                       factor with X X^T = J^-1.

Pinned by tests/test_oracle_df_mp2.py: the energy is unchanged when the
auxiliary basis is rotated (eri -> eri Q, J -> Q^T J Q, Q orthogonal: the
energy sees J only through J^-1 contracted with the three-index tensor; a
transposed factor, B = (ia|P) X^T, breaks it), unchanged when L^-T is
replaced by the symmetric J^-1/2, and equal to the pair energy of the eri
block itself when J = I and the orbitals are columns of the identity.
"""

from __future__ import annotations

import numpy as np
import torch

from . import metric, pair_energy


def inv_sqrt_sym(J) -> np.ndarray:
    w, V = np.linalg.eigh(np.asarray(J, dtype=np.float64))
    return (V / np.sqrt(w)) @ V.T


def df_mp2_energy_ref(C_occ, C_vir, eri, J, eps_occ, eps_vir, factor=None) -> float:
    C_occ, C_vir, eri, J = (np.asarray(x, dtype=np.float64) for x in (C_occ, C_vir, eri, J))
    X = metric.metric_inv_half_ref(J) if factor is None else np.asarray(factor, dtype=np.float64)
    iv = np.einsum("mi,mnP->inP", C_occ, eri)
    ia = np.einsum("na,inP->iaP", C_vir, iv)
    B = ia @ X
    return pair_energy.pair_energy_f64(
        torch.from_numpy(B), torch.as_tensor(np.asarray(eps_occ, dtype=np.float64)),
        torch.as_tensor(np.asarray(eps_vir, dtype=np.float64)),
    )  # fmt: skip
