"""GPU values of the torch.ops.trnblas.* surface (reference layouts and
result shapes) against the oracle."""

import numpy as np
import pytest
import torch

from oracle import ozaki as oz
from oracle import pair_energy as pe
from trnblas_amd import df_mp2
from trnblas_amd.hip import get_native_ops

pytestmark = pytest.mark.gpu


def test_gemm_ops(dev):
    ops = get_native_ops()
    g = torch.Generator(device=dev).manual_seed(0)
    a = torch.randn(256, 128, device=dev, generator=g)
    b = torch.randn(128, 200, device=dev, generator=g)
    ref = a.double() @ b.double()
    for name in ("gemm_128_128_512", "gemm_64_128_128", "gemm_ragged", "gemm_lnc"):
        assert (ops[name](a, b).double() - ref).abs().max() < 1e-3
    assert (ops["gemm_lnc_tn"](a.T.contiguous(), b).double() - ref).abs().max() < 1e-3
    s = ops["syrk"](a)
    assert torch.equal(s, s.T) and (s.double() - a.double() @ a.double().T).abs().max() < 1e-3


def test_energy_ops(dev):
    ops = get_native_ops()
    B, eo, ev = df_mp2.pair_inputs(5, 128, 256, dev, seed=1)
    evc, evr = ev.reshape(-1, 1), ev.reshape(1, -1)
    full = pe.pair_energy_f64(B, eo, ev)
    out = ops["batched_pair"](B, eo.reshape(1, -1), evc, evr)
    assert out.shape == (128, 25) and abs(float(out.double().sum()) - full) <= 1e-6 * abs(full)
    out = ops["j_batched"](B[2], B, eo[2:3].reshape(1, 1), eo.reshape(1, -1), evc, evr)
    want = pe.pair_energies_f64(B, B, eo, eo, ev, [(2, j) for j in range(5)])
    assert torch.allclose(out.double().sum(0).cpu(), want, rtol=1e-6)
    # the reference's per-row window: j = i + d (mod nocc), B[j]^T operands
    i, nd = 1, 4
    js = [(i + dd) % 5 for dd in range(nd)]
    Bt = B.transpose(1, 2).contiguous()
    out = ops["pair_energy_sym"](Bt[i], Bt[js], eo[i : i + 1].reshape(1, 1), eo[js].reshape(1, -1), evc, evr)
    want = pe.pair_energies_f64(B, B, eo, eo, ev, [(i, j) for j in js])
    assert out.shape == (128, nd) and torch.allclose(out.double().sum(0).cpu(), want, rtol=1e-6)
    eos = (eo[0] + eo[3]).reshape(1, 1)
    out = ops["fused_gemm_energy"](B[0], B[3], eos, evc, evr)
    want = pe.pair_energies_f64(B, B, eo, eo, ev, [(0, 3)])
    assert out.shape == (128, 1) and abs(float(out.double().sum()) - float(want[0])) <= 1e-6 * abs(float(want[0]))
    flat = B.reshape(5 * 128, 256)
    T_flat = flat[:256] @ flat.T
    out = ops["mp2_energy"](T_flat, eo[:2].reshape(1, -1), eo.reshape(1, -1), evc, evr)
    want = float(pe.mp2_energy_cpu(T_flat.double().cpu(), eo[:2].double().cpu(), eo.double().cpu(), ev.double().cpu()))
    assert out.shape == (128, 10) and abs(float(out.double().sum()) - want) <= 1e-6 * abs(want)


def test_ozaki_ops(dev):
    ops = get_native_ops()
    rng = np.random.default_rng(3)
    X = rng.standard_normal((70, 150)) * 10.0 ** rng.uniform(-5, 5, (70, 150))
    xw = torch.from_numpy(X).view(torch.int32).to(dev)
    emax = ops["ozaki_emax"](xw).cpu().numpy()[:, 0]
    want = ((X.view(np.uint64) >> np.uint64(52)) & np.uint64(0x7FF)).max(axis=1)
    assert np.array_equal(emax, want.astype(np.float32))
    emc = ops["ozaki_emax_col"](xw).cpu().numpy()[0]
    assert np.array_equal(emc, ((X.view(np.uint64) >> np.uint64(52)) & np.uint64(0x7FF)).max(axis=0).astype(np.float32))
    k = 8
    d = ops["ozaki_split"](xw, torch.zeros(128, k, device=dev))
    dw, _ = oz.split(X, k, per="row", pad=(128, 128))
    assert d.shape == (k, 128, 256) and np.array_equal(d.float().cpu().numpy(), dw.astype(np.float32))
    d = ops["ozaki_split_col"](xw, torch.zeros(k, 256, device=dev))
    dw, _ = oz.split(X, k, per="col", pad=(128, 128))
    assert np.array_equal(d.float().cpu().numpy(), dw.astype(np.float32))
    # slice GEMM (hi, lo) in the reference layout (k, Kp, Mp) x (k, Kp, N)
    A = rng.standard_normal((50, 300))
    B = rng.standard_normal((300, 40))
    at, _ = oz.split_a(A, k)
    bt, _ = oz.split_b(B, k)
    hl = ops["ozaki_gemm"](torch.from_numpy(at).to(dev).bfloat16(), torch.from_numpy(bt[:, :, :40]).to(dev).bfloat16())
    want = oz.reference_from_digits(at, bt[:, :, :40])
    assert hl.shape == want.shape and np.array_equal(hl.cpu().numpy().view(np.int32), want.view(np.int32))
