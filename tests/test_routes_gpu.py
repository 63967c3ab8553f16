"""The routes of the public API on the GPU box: host operands large enough
for the upload route (the reference's `_upload` / `_to_host`,
nki/dispatch.py:254-274, :2075-2101) come back on the host in pinned memory
and match the reference's CPU path at 1e-6 |A||B|; device-resident calls
take the kernel or hipBLASLt as the measured crossover says (the
reference's `_gemm_route` / `_lnc_gemm_wins`, :633-727), and the pair energy
takes the fused kernel or the unfused path by its crossover (:2680-2703)."""

import pytest
import torch

import trnblas_amd as tb
from oracle import blas
from oracle import pair_energy as pe
from trnblas_amd import df_mp2
from trnblas_amd.hip import dispatch as d
from trnblas_amd.hip import kernels

pytestmark = pytest.mark.gpu


def _cw(D, ref, den):
    den = torch.where(den > 0, den, torch.ones_like(den))
    return float(((D.double() - ref) / den).abs().max())


class _Launches:
    """Names of the HIP kernel families launched while active."""

    def __init__(self):
        self.names = []

    def __call__(self, kernel, phase):
        if phase == "begin":
            self.names.append(kernel)

    def __enter__(self):
        kernels._launch_probe = self
        return self

    def __exit__(self, *exc):
        kernels._launch_probe = None


def test_upload_route_gemm_batched_syrk(dev):
    g = torch.Generator().manual_seed(21)
    A = torch.randn(2048, 1536, generator=g)
    B = torch.randn(1536, 1024, generator=g)
    C = torch.randn(2048, 1024, generator=g)
    assert d._gemm_route(A, B) == "upload"
    with _Launches() as seen:
        D = tb.gemm(1.0, A, B, beta=0.5, C=C)
    assert "gemm" in seen.names  # the kernel ran on the GPU
    assert D.device.type == "cpu" and D.is_pinned()
    den = blas.gemm_cw_den(1.0, A, B, 0.5, C)
    assert _cw(D, blas.gemm_cpu(1.0, A, B, 0.5, C).double(), den) <= 1e-6
    assert _cw(D, blas.gemm_f64(1.0, A, B, 0.5, C), den) <= 1e-6

    A3 = torch.randn(8, 512, 1024, generator=g)
    B3 = torch.randn(8, 1024, 512, generator=g)
    assert d._gemm_route(A3, B3, op="batched_gemm") == "upload"
    with _Launches() as seen:
        D3 = tb.batched_gemm(1.0, A3, B3)
    assert "gemm" in seen.names
    assert D3.device.type == "cpu" and D3.is_pinned()
    ref3 = A3.double() @ B3.double()
    assert _cw(D3, ref3, A3.double().abs() @ B3.double().abs()) <= 1e-6

    # TRNBLAS_PINNED_OUTPUT=0 (nki/dispatch.py:2052-2060): pageable results
    import os

    os.environ["TRNBLAS_PINNED_OUTPUT"] = "0"
    try:
        D0 = tb.gemm(1.0, A, B, beta=0.5, C=C)
    finally:
        del os.environ["TRNBLAS_PINNED_OUTPUT"]
    assert D0.device.type == "cpu" and not D0.is_pinned() and torch.equal(D0, D)

    As = torch.randn(1536, 2048, generator=g)
    X = torch.randn(1536, 1536, generator=g)
    Cs = torch.tril(X) + torch.tril(X, -1).T
    with _Launches() as seen:
        S = tb.syrk(1.0, As, beta=0.5, C=Cs, uplo="lower")
    assert "syrk" in seen.names
    assert S.device.type == "cpu" and S.is_pinned() and torch.equal(S, S.T)
    ref = blas.syrk_f64(1.0, As, 0.5, Cs, uplo="lower")
    den = As.double().abs() @ As.double().abs().T + 0.5 * Cs.double().abs()
    assert _cw(S, ref, den) <= 1e-6
    assert _cw(S, blas.syrk_cpu(1.0, As, 0.5, Cs, uplo="lower").double(), den) <= 1e-6


def test_device_gemm_route_by_dtype_and_shape(dev):
    g = torch.Generator(device=dev).manual_seed(22)
    # fp32: the kernel at every size (the 1e-6 gate)
    A = torch.randn(4096, 4096, device=dev, generator=g)
    with _Launches() as seen:
        D = tb.gemm(1.0, A, A)
    assert seen.names == ["gemm"]
    # bf16 at 4096^3: hipBLASLt (measured 0.77-0.87 of the kernel's time)
    Ab = A.bfloat16()
    with _Launches() as seen:
        Db = tb.gemm(1.0, Ab, Ab)
    assert seen.names == []
    ref = (Ab.float() @ Ab.float()).double()
    den = Ab.float().abs() @ Ab.float().abs()
    assert _cw(Db.float(), ref, den.double()) <= 2.0**-8
    # bf16 with a short K: the kernel
    As, Bs = Ab[:, :128].contiguous(), Ab[:128].contiguous()
    with _Launches() as seen:
        tb.gemm(1.0, As, Bs)
    assert seen.names == ["gemm"]
    # bf16 SYRK: always the kernel (the triangle)
    with _Launches() as seen:
        tb.syrk(1.0, Ab[:2048])
    assert seen.names == ["syrk"]
    del A, D, Ab, Db


def test_pair_energy_route_small_shape_takes_unfused(dev):
    B, eo, ev = df_mp2.pair_inputs(2, 448, 1536, seed=23)
    Bd, eod, evd = B.to(dev), eo.to(dev), ev.to(dev)
    assert d._pair_energy_route(Bd) == "aten"
    with _Launches() as seen:
        e = d.nki_batched_pair_energy(Bd, eod, evd)
    assert "pair_energy" not in seen.names
    want = pe.pair_energy_f64(B, eo, ev)
    assert abs(float(e) - want) <= 1e-6 * abs(want)
    # and the fused kernel on the same inputs agrees
    got = float(kernels.pair_energy_sym(Bd, eod, evd))
    assert abs(got - want) <= 1e-6 * abs(want)


def test_autotune_measures_once_per_bucket(dev, monkeypatch, tmp_path):
    # with autotune on, the first 16-bit device GEMM of a shape bucket times
    # the kernel and hipBLASLt and routes by the result; later calls of the
    # bucket reuse it (also from the cache file), fp32 is never timed
    path = tmp_path / "autotune.json"
    monkeypatch.setattr(d, "_AUTOTUNE_CACHE_FILE", str(path))
    monkeypatch.setattr(d, "_autotune_mem", {})
    monkeypatch.setattr(d, "_autotune_loaded", False)
    monkeypatch.setattr(d, "_autotune_measured", 0)
    monkeypatch.setattr(d, "_AUTOTUNE", True)
    g = torch.Generator(device=dev).manual_seed(31)
    A = torch.randn(2048, 1024, device=dev, generator=g).bfloat16()
    B = torch.randn(1024, 1536, device=dev, generator=g).bfloat16()
    route = d._gemm_route(A, B)
    assert route in ("hip", "aten") and d._autotune_measured == 1
    key = d._autotune_key(A.shape, B.shape, A.dtype, False, False, True)
    assert d._autotune_mem[key] == route
    import json

    assert json.loads(path.read_text())[key] == route
    with _Launches() as seen:
        D = tb.gemm(1.0, A, B)
    assert ("gemm" in seen.names) == (route == "hip")
    ref = A.double() @ B.double()
    den = A.double().abs() @ B.double().abs()
    assert _cw(D, ref, den) <= 2.0**-8
    # a shape of the same bucket, and a fresh process state reading the file
    A2, B2 = A[:1500, :1000].contiguous(), B[:1000, :1100].contiguous()
    assert d._gemm_route(A2, B2) == route and d._autotune_measured == 1
    monkeypatch.setattr(d, "_autotune_mem", {})
    monkeypatch.setattr(d, "_autotune_loaded", False)
    assert d._gemm_route(A, B) == route and d._autotune_measured == 1
    # fp32 stays on the kernel without a measurement
    assert d._gemm_route(A.float(), B.float()) == "hip" and d._autotune_measured == 1


def test_unready_16bit_routes_to_hipblaslt(dev):
    # bf16 operands the DMA kernel cannot read in place (K = 1023), below the
    # hipBLASLt shape bucket: hipBLASLt from 2^26 multiply-adds, the kernel
    # below; both within the 16-bit gate
    g = torch.Generator(device=dev).manual_seed(31)
    for n, launches in ((1023, []), (255, ["gemm"])):
        A = torch.randn(n, n, device=dev, generator=g).bfloat16()
        B = torch.randn(n, n, device=dev, generator=g).bfloat16()
        with _Launches() as seen:
            D = tb.gemm(1.0, A, B)
        assert seen.names == launches
        ref = A.double() @ B.double()
        den = A.double().abs() @ B.double().abs()
        assert _cw(D.double(), ref, den) <= 2.0**-8


@pytest.mark.parametrize(
    "M,N,K,tra,trb", [(2048, 2048, 2048, True, False), (300, 260, 128, False, True), (64, 64, 64, True, True),
                    (130, 68, 4100, False, False)],
)
def test_gemm_fast_path_equals_general_path(dev, monkeypatch, M, N, K, tra, trb):
    # the public 2-D fp32 gemm on device operands skips the general routing;
    # its result is the library call's, bit for bit, and it never reaches
    # gemm_scaled
    g = torch.Generator().manual_seed(M + N + K)
    A = torch.randn((K, M) if tra else (M, K), generator=g).to(dev)
    B = torch.randn((N, K) if trb else (K, N), generator=g).to(dev)
    C = torch.randn(M, N, generator=g).to(dev)
    want = kernels.gemm(A.mT if tra else A, B.mT if trb else B, 0.75, 0.5, C)

    def refuse(*a, **k):
        raise AssertionError("general path taken")

    monkeypatch.setattr(d, "gemm_scaled", refuse)
    D = tb.gemm(0.75, A, B, beta=0.5, C=C, transA=tra, transB=trb)
    torch.cuda.synchronize()
    assert torch.equal(D, want)
    D0 = tb.gemm(1.0, A, B, transA=tra, transB=trb)  # no C
    assert torch.equal(D0, kernels.gemm(A.mT if tra else A, B.mT if trb else B))


def test_gemm_fast_path_declines(dev, monkeypatch):
    # every case the fast path does not take reaches the general path, with
    # the general path's result
    g = torch.Generator().manual_seed(5)
    A = torch.randn(96, 80, generator=g).to(dev)
    B = torch.randn(80, 72, generator=g).to(dev)
    C = torch.randn(96, 72, generator=g).to(dev)
    taken = []
    general = d.gemm_scaled

    def spy(*a, **k):
        taken.append(1)
        return general(*a, **k)

    monkeypatch.setattr(d, "gemm_scaled", spy)
    ref = A.double() @ B.double()
    den = A.double().abs() @ B.double().abs()
    cases = [
        lambda: tb.gemm(1.0, A, B, beta=0.5, C=C[:1].expand(96, 72)),  # broadcast C view
        lambda: tb.gemm(1.0, A[:, 1:], B[1:]),  # 4-byte aligned base, K = 79
        lambda: tb.gemm(1.0, A.half(), B.half()),  # not fp32
        lambda: tb.gemm(1.0, A, B, transA="N"),  # a string flag
    ]
    for i, fn in enumerate(cases):
        n0 = len(taken)
        D = fn()
        assert len(taken) == n0 + 1, i
        assert D.shape[0] == 96
    Ag = A.clone().requires_grad_(True)
    n0 = len(taken)
    D = tb.gemm(1.0, Ag, B)
    assert len(taken) == n0 + 1 and D.requires_grad
    monkeypatch.setenv("TRNBLAS_NATIVE_GEMM", "aten")
    n0 = len(taken)
    D = tb.gemm(1.0, A, B)
    assert len(taken) == n0 + 1
    assert (((D.double() - ref).abs() / den).max()) <= 1e-6
