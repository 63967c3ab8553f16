"""Config 5 (gemm_fp64 8192^3 on C5's wide-range data) across slice counts,
judged over the whole 8192 x 8192 output.

The judge is oracle.exact.ref_exact (the restated judge of the reference's
tests/_ozaki_ref.py:16-48), evaluated on the device: its slice products are
exact in any fp64 GEMM, so the device form has the numpy form's bits
(checked here on sample rows).

The reference's gate for host-fp64 accuracy on wide-range data
(tests/test_ozaki.py:190-194, tests/_ozaki_ref.py:51-56):
    max |C - C_exact| / (|A||B|) <= max(4 host, 4e-15)
over every element, host being the same measure of the host CPU's fp64 BLAS
product A @ B. Every k must also stay within the a-priori k-slice bound.
The smallest k that meets the gate on this data is HOST_ACCURATE_SLICES; the
test asserts that k exactly (it fails if a change makes a smaller k pass or
that k fail)."""

import numpy as np
import pytest
import torch

import trnblas_amd as tb
from oracle import exact
from oracle import ozaki as oz
from trnblas_amd import df_mp2

pytestmark = pytest.mark.gpu

HOST_ACCURATE_SLICES = 11
ROWS = [0, 1001, 2048, 3333, 4095, 5000, 6143, 7777, 8190, 8191]


@pytest.fixture(scope="module")
def c5():
    from conftest import gpu_ready

    if not gpu_ready():
        pytest.skip("no ROCm GPU")
    dev = torch.device("cuda", 0)
    n = 8192
    A, B = df_mp2.config5_inputs(dev, n, seed=5)
    ex = exact.ref_exact(A, B, xp=torch)
    # the device judge has the numpy judge's bits
    ex_rows = exact.ref_exact(A[ROWS].cpu().numpy(), B.cpu().numpy())
    assert np.array_equal(ex[ROWS].cpu().numpy().view(np.int64), ex_rows.view(np.int64))
    den = A.abs() @ B.abs()
    den = torch.where(den > 0, den, torch.ones_like(den))
    host = (A.cpu() @ B.cpu()).to(dev)  # the host CPU's fp64 BLAS, as the reference's gate
    return A, B, ex, den, host


def _cw(C, ex, den) -> float:
    return float(((C - ex).abs() / den).max())


def test_config5_slice_sweep_full_matrix(c5):
    A, B, ex, den, host_C = c5
    n = A.shape[1]
    host = _cw(host_C, ex, den)
    dgemm = _cw(A @ B, ex, den)  # the device's native fp64 DGEMM, reported
    gate = max(4 * host, 4e-15)
    errs = {}
    for k in range(8, 13):
        C = tb.gemm_fp64(A, B, slices=k, mode="fast")
        errs[k] = _cw(C, ex, den)
        # within the k-slice bound (plus fp64 rounding of the recombination)
        bound = oz.error_bound(A, B, k, absA_absB=den, xp=torch) + n * 2.0**-53 * den
        assert bool(((C - ex).abs() <= bound).all()), k
        del C, bound
    meets = [k for k, e in errs.items() if e <= gate]
    print(f"config5 full 8192^2: host BLAS {host:.3e}, device DGEMM {dgemm:.3e}, gate {gate:.3e}, "
          + ", ".join(f"k={k}: {e:.3e}" for k, e in errs.items())
          + f"; smallest k at host accuracy: {meets[0] if meets else None}", flush=True)
    # each added slice shrinks the truncation by 2^-7 until the fp64 floor
    for k in range(8, 12):
        assert errs[k + 1] <= max(errs[k] / 16, 4 * host), (k, errs)
    assert meets and meets[0] == HOST_ACCURATE_SLICES, (gate, errs)
    assert all(errs[k] <= gate for k in range(HOST_ACCURATE_SLICES, 13)), (gate, errs)


def test_config5_exact_mode_host_accurate_slices(c5):
    """The bit-exact mode (the reference's own arithmetic) at the same k."""
    A, B, ex, den, host_C = c5
    gate = max(4 * _cw(host_C, ex, den), 4e-15)
    C = tb.gemm_fp64(A, B, slices=HOST_ACCURATE_SLICES, mode="exact")
    err = _cw(C, ex, den)
    print(f"config5 exact mode k={HOST_ACCURATE_SLICES}: {err:.3e} (gate {gate:.3e})", flush=True)
    bound = oz.error_bound(A, B, HOST_ACCURATE_SLICES, absA_absB=den, xp=torch)
    assert bool(((C - ex).abs() <= bound + A.shape[1] * 2.0**-53 * den).all())
    assert err <= gate, (err, gate)


def test_config5_crt_mode_host_accuracy(c5):
    """Scheme II (mode "crt") on the same data and gate: no digit products are
    dropped, so at equal k it is at least as accurate as the digit split."""
    A, B, ex, den, host_C = c5
    n = A.shape[1]
    gate = max(4 * _cw(host_C, ex, den), 4e-15)
    errs = {}
    for k in (9, 10, 11, 12):
        C = tb.gemm_fp64(A, B, slices=k, mode="crt")
        errs[k] = _cw(C, ex, den)
        bound = oz.error_bound(A, B, k, absA_absB=den, xp=torch) + n * 2.0**-53 * den
        assert bool(((C - ex).abs() <= bound).all()), k
        del C, bound
    meets = [k for k, e in errs.items() if e <= gate]
    print(f"config5 crt mode: gate {gate:.3e}, " + ", ".join(f"k={k}: {e:.3e}" for k, e in errs.items())
          + f"; smallest k at host accuracy: {meets[0] if meets else None}", flush=True)
    assert meets and meets[0] <= HOST_ACCURATE_SLICES, errs
    assert all(errs[k] <= gate for k in range(meets[0], 13)), errs
