"""The example's whole DF-MP2 calculation on the MI355X: metric factor on the
device (HIP diagonal-block kernel + DGEMMs), half-transforms and metric
contraction on the HIP GEMM kernels, each energy path on its HIP kernel,
against the float64 chain oracle. Gate: relative 1e-6 (north star)."""

import pytest

from oracle import df_mp2 as od
from trnblas_amd import df_mp2

pytestmark = pytest.mark.gpu

PATHS = [{}, {"use_fused": True}, {"use_fused_gemm": True}, {"use_batched_pair": True}]


@pytest.mark.parametrize("kw", PATHS, ids=["chunked", "fused", "fused_gemm", "batched_pair"])
@pytest.mark.parametrize("shape", [(48, 6, 80), (96, 8, 200)])
def test_df_mp2_energy_device_paths(dev, kw, shape):
    inp = df_mp2.make_inputs(*shape, seed=5)
    want = od.df_mp2_energy_ref(*(t.double().numpy() for t in inp))
    t = {}
    e = df_mp2.df_mp2_energy(*(x.to(dev) for x in inp), timings=t, **kw)
    assert abs(e - want) <= 1e-6 * abs(want), (e, want)
    assert all(v >= 0.0 for v in t.values())
