"""The example's whole DF-MP2 calculation (trnblas_amd.df_mp2.df_mp2_energy,
examples/df_mp2.py:147-233) on host tensors (torch: the reference's own host
route) against the float64 chain oracle. Gate: relative 1e-6 (north star)."""

import numpy as np
import pytest

from oracle import df_mp2 as od
from trnblas_amd import df_mp2

PATHS = [{}, {"use_fused": True}, {"use_fused_gemm": True}, {"use_batched_pair": True}]


@pytest.mark.parametrize("kw", PATHS, ids=["chunked", "fused", "fused_gemm", "batched_pair"])
def test_df_mp2_energy_host_paths(kw):
    inp = df_mp2.make_inputs(24, 4, 40, seed=3)
    want = od.df_mp2_energy_ref(*(t.double().numpy() for t in inp))
    t = {}
    e = df_mp2.df_mp2_energy(*inp, timings=t, **kw)
    assert abs(e - want) <= 1e-6 * abs(want), (e, want)
    assert set(t) == {"chol", "half", "metric", "energy"}


def test_make_inputs_and_flops():
    # the example's recipe: seeded global generator, documented shapes,
    # J = J_raw J_raw^T + naux I (SPD), sorted orbital energies
    a = df_mp2.make_inputs(16, 3, 20, seed=9)
    b = df_mp2.make_inputs(16, 3, 20, seed=9)
    for x, y in zip(a, b):
        assert np.array_equal(x.numpy(), y.numpy())
    C_occ, C_vir, eri, J, eo, ev = a
    assert C_occ.shape == (16, 3) and C_vir.shape == (16, 13) and eri.shape == (16, 16, 20)
    assert J.shape == (20, 20) and np.linalg.eigvalsh(J.double().numpy()).min() > 0
    assert np.all(np.diff(eo.numpy()) <= 0) and eo.max() < -0.5
    assert np.all(np.diff(ev.numpy()) >= 0) and ev.min() > 0.1
    # flops of (8, 2, 4): 2a 2*64*2*4 + 2b 2*2*6*8*4 + 3 2*2*6*16 + 4 2*4*36*4
    assert df_mp2.flops(8, 2, 4) == 1024 + 768 + 384 + 1152


def test_bench_harness_shapes_and_cli(capsys):
    # the example's bench shapes and harness (examples/df_mp2.py:269-333)
    assert df_mp2.BENCH_SHAPES == {"small": (128, 16, 384), "medium": (512, 64, 1536),
                                   "large": (768, 96, 2304)}
    assert df_mp2.BENCH_SHAPES["large"][0] - df_mp2.BENCH_SHAPES["large"][1] == 672  # C3's nvir
    rows = df_mp2.bench("small", passes="both", use_batched_pair=True, verbose=False)
    assert [r["pass_"] for r in rows] == ["cold", "warm"]
    inp = df_mp2.make_inputs(*df_mp2.BENCH_SHAPES["small"])
    want = od.df_mp2_energy_ref(*(t.double().numpy() for t in inp))
    for r in rows:
        assert abs(r["E"] - want) <= 1e-6 * abs(want)
        assert r["tflops"] > 0 and {"chol", "half", "metric", "energy"} <= set(r)
    df_mp2.main(["--demo", "--fused-energy"])
    assert "E_MP2" in capsys.readouterr().out
