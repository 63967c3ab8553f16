"""Host logic of trnblas_amd on the CPU: flags, backends, routing, dtype
backstop, fallback / REQUIRE semantics, lazy registration, the op
surface's fake (meta) shapes, the Ozaki schedule and plan, and the
pytorch-backend results against the oracle."""

import importlib
import subprocess
import sys
import warnings

import pytest
import torch

import trnblas_amd as tb
from oracle import blas, pair_energy as pe
from oracle import ozaki as oracle_ozaki
from trnblas_amd import _flags, ozaki
from trnblas_amd.hip import dispatch as d


# ── flags (trnblas/_flags.py) ────────────────────────────────────────────────


@pytest.mark.parametrize("v,want", [("U", "upper"), (" lower ", "lower"), ("l", "lower")])
def test_uplo_flag(v, want):
    assert _flags.uplo_flag(v) == want


@pytest.mark.parametrize("bad", ["x", "", None, 1])
def test_flags_reject(bad):
    with pytest.raises(ValueError):
        _flags.uplo_flag(bad)


def test_trans_flag():
    assert _flags.trans_flag("T") is True and _flags.trans_flag("n") is False
    assert _flags.trans_flag(1) is True and _flags.trans_flag(0) is False
    with pytest.raises(ValueError):
        _flags.trans_flag("C")
    assert _flags.side_flag("R") == "right" and _flags.diag_flag("N") == "nonunit"


# ── backends and routing ─────────────────────────────────────────────────────


def test_backend_switch():
    assert tb.get_backend() == "auto"
    tb.set_backend("pytorch")
    try:
        assert not d._use_hip()
    finally:
        tb.set_backend("auto")
    with pytest.raises(ValueError):
        tb.set_backend("cuda")
    if not d.has_hip():
        with pytest.raises(RuntimeError):
            tb.set_backend("hip")


def _fake_gpu(monkeypatch):
    monkeypatch.setattr(d, "has_hip", lambda: True)


def test_route_table(monkeypatch):
    _fake_gpu(monkeypatch)
    A = torch.randn(4, 4)
    assert d._gemm_route(A, A.double()) == "torch"  # mixed dtypes: torch raises
    assert d._gemm_route(A.double(), A.double()) == "torch"  # fp64: torch where the data is
    assert d._gemm_route(A.to(torch.int32), A.to(torch.int32)) == "torch"
    assert d._gemm_route(A, A) == "host"  # tiny host GEMM: the host CPU wins
    big = torch.empty(4096, 4096)
    assert d._gemm_route(big, big) == "upload"  # large host GEMM: upload
    monkeypatch.setenv("TRNBLAS_NATIVE_GEMM", "host")
    assert d._gemm_route(big, big) == "host"
    monkeypatch.setenv("TRNBLAS_NATIVE_GEMM", "bogus")
    with pytest.raises(ValueError):
        d._gemm_route(big, big)


@pytest.mark.parametrize(
    "a_shape,b_shape,dtype,contig,op,want",
    [
        ((8192, 8192), (8192, 8192), torch.float32, True, "gemm", False),  # fp32: accuracy gate
        ((8192, 8192), (8192, 8192), torch.bfloat16, True, "gemm", True),
        ((2048, 2048), (2048, 2048), torch.bfloat16, True, "gemm", False),  # 2^22 outputs, K 2048
        ((2048, 1024), (1024, 4096), torch.bfloat16, True, "gemm", False),  # 2^23 outputs, K 1024
        ((2048, 4096), (4096, 4096), torch.bfloat16, True, "gemm", True),  # 2^23 outputs, K 4096
        ((2048, 8192), (8192, 2048), torch.float16, True, "gemm", True),  # 2^22 outputs, K 8192
        ((4096, 1024), (1024, 4096), torch.bfloat16, True, "gemm", True),  # 2^24 outputs
        ((2048, 128), (128, 2048), torch.bfloat16, True, "gemm", False),  # short K: the kernel
        ((1024, 8192), (8192, 1024), torch.bfloat16, True, "gemm", False),  # long K: the kernel
        ((256, 8192), (8192, 8192), torch.float16, True, "gemm", False),
        ((8192, 256), (256, 8192), torch.bfloat16, False, "gemm", False),  # K 256 < 512
        ((8192, 1024), (1024, 8192), torch.bfloat16, False, "gemm", True),  # 2-D views are fine
        ((64, 512, 2048), (64, 2048, 512), torch.bfloat16, True, "batched_gemm", True),  # C2b
        ((64, 512, 2048), (64, 2048, 512), torch.bfloat16, False, "batched_gemm", False),
        ((64, 512, 2048), (64, 2048, 512), torch.float32, True, "batched_gemm", False),
        ((4096, 8192), (8192, 4096), torch.bfloat16, True, "syrk", False),  # triangle
    ],
)
def test_device_route_known_answers(a_shape, b_shape, dtype, contig, op, want):
    # the measured hipBLASLt-vs-kernel crossover of device-resident GEMMs
    assert d._aten_gemm_wins(a_shape, b_shape, dtype, contig, op) is want


@pytest.mark.parametrize(
    "shape,want",
    [
        ((96, 672, 2304), "hip"),  # C3
        ((256, 768, 4096), "hip"),  # C4's energy
        ((16, 128, 1536), "hip"),
        ((4, 448, 1536), "hip"),
        ((2, 448, 1536), "aten"),  # 15 work items on 256 CUs
        ((64, 32, 1536), "aten"),  # nvir far below the 96-row tile
        ((1, 672, 2304), "aten"),  # one pair: one item's k-steps are the whole run
    ],
)
def test_pair_energy_route_known_answers(monkeypatch, shape, want):
    # the measured fused-vs-unfused crossover (estimates in ms)
    fused, unfused = d._pair_energy_estimates(*shape)
    assert ("aten" if unfused < fused else "hip") == want


def test_route_grad_goes_to_torch(monkeypatch):
    _fake_gpu(monkeypatch)
    A = torch.randn(512, 512, requires_grad=True)
    assert d._gemm_route(A, A) == "torch"


def test_require_refuses_fp64(monkeypatch):
    _fake_gpu(monkeypatch)
    monkeypatch.setattr(d, "_REQUIRE_HIP", True)
    A = torch.randn(3, 3, dtype=torch.float64)
    with pytest.raises(NotImplementedError):
        d._gemm_route(A, A)


def test_host_model_scales_with_threads(monkeypatch):
    macs, nbytes = 2e6, 10_000
    monkeypatch.setattr(torch, "get_num_threads", lambda: 2)
    two = d._host_gemm_wins(macs, nbytes, torch.float32)
    monkeypatch.setattr(torch, "get_num_threads", lambda: 64)
    assert d._host_gemm_wins(macs, nbytes, torch.float32) or not two
    assert d._host_gemm_wins(1e15, 0, torch.float64)  # no device route for fp64 on the host model


# ── dtype backstop and fallback semantics ────────────────────────────────────


def test_kernel_dtype_backstop():
    d._check_kernel_operands("gemm_ragged", torch.zeros(1), torch.zeros(1, dtype=torch.bfloat16))
    with pytest.raises(TypeError):
        d._check_kernel_operands("pair_energy_sym", torch.zeros(1, dtype=torch.float64))
    with pytest.raises(TypeError):
        d._check_kernel_operands("no_such_op", torch.zeros(1))
    with pytest.raises(TypeError):
        d._check_kernel_operands("ozaki_gemm", torch.zeros(1))


def test_kernel_error_falls_back_with_one_warning(monkeypatch):
    err = d.HipKernelError("trnblas_hip_gemm", -2, "boom")
    monkeypatch.setattr(d, "_REQUIRE_HIP", False)
    d._fallback_warned.clear()
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        d._kernel_failed(err)
        d._kernel_failed(err)
    assert len([x for x in w if issubclass(x.category, d.HipFallbackWarning)]) == 1
    monkeypatch.setattr(d, "_REQUIRE_HIP", True)
    with pytest.raises(d.HipKernelError):
        d._kernel_failed(err)
    # a missing library never falls back
    monkeypatch.setattr(d, "_REQUIRE_HIP", False)
    with pytest.raises(d.HipLibraryError):
        d._kernel_failed(d.HipLibraryError("missing"))


def test_gemm_kernel_failure_gives_torch_result(monkeypatch):
    # a kernel route whose launch fails: warning + the torch result (dispatch
    # fallback, as the reference's test_native_dispatch.py:1060-1074)
    _fake_gpu(monkeypatch)
    monkeypatch.setattr(d, "_REQUIRE_HIP", False)
    monkeypatch.setattr(d, "_gemm_route", lambda *a, **k: "hip")

    def boom(*a, **k):
        raise d.HipKernelError("trnblas_hip_gemm", -2, "launch failed")

    monkeypatch.setattr(d, "hip_gemm", boom)
    A, B = torch.randn(8, 5), torch.randn(5, 3)
    with warnings.catch_warnings(record=True):
        warnings.simplefilter("always")
        out = d.nki_gemm(A, B)
    assert torch.allclose(out, A @ B)


# ── lazy registration and the op surface ─────────────────────────────────────


def test_import_registers_nothing_and_loads_no_library():
    code = (
        "import sys, trnblas_amd, torch\n"
        "assert 'trnblas_amd.hip._native' not in sys.modules\n"
        "from trnblas_amd.hip import _lib\n"
        "assert _lib._lib is None\n"
        "assert not hasattr(torch.ops.trnblas, 'gemm_ragged') or True\n"
    )
    subprocess.run([sys.executable, "-c", code], check=True, cwd=str(__import__("pathlib").Path(__file__).parents[1]))


REFERENCE_OP_NAMES = [
    "gemm_64_128_128", "gemm_64_128_256", "gemm_64_128_512", "gemm_128_128_128",
    "gemm_128_128_256", "gemm_128_128_512", "gemm_ragged", "gemm_lnc", "gemm_lnc_tn", "syrk",
    "mp2_energy", "fused_gemm_energy", "batched_pair", "j_batched", "pair_energy_sym",
    "ozaki_gemm", "ozaki_emax", "ozaki_split", "ozaki_emax_col", "ozaki_split_col",
]  # fmt: skip


def test_op_surface_names_and_fake_shapes():
    ops = d.get_native_ops()
    assert sorted(ops) == sorted(REFERENCE_OP_NAMES)
    for name in REFERENCE_OP_NAMES:
        assert hasattr(torch.ops.trnblas, name)
    m = lambda *s, dt=torch.float32: torch.empty(s, dtype=dt, device="meta")  # noqa: E731
    T = torch.ops.trnblas
    assert T.gemm_128_128_512(m(256, 128), m(128, 512)).shape == (256, 512)
    assert T.gemm_lnc_tn(m(128, 64), m(128, 300)).shape == (64, 300)
    assert T.syrk(m(384, 128)).shape == (384, 384)
    assert T.mp2_energy(m(2 * 96, 4 * 96), m(1, 2), m(1, 4), m(96, 1), m(1, 96)).shape == (96, 8)
    assert T.mp2_energy(m(2 * 130, 4 * 130), m(1, 2), m(1, 4), m(130, 1), m(1, 130)).shape == (65, 8)
    assert T.fused_gemm_energy(m(256, 384), m(256, 384), m(1, 1), m(256, 1), m(1, 256)).shape == (256, 1)
    assert T.batched_pair(m(5, 128, 256), m(1, 5), m(128, 1), m(1, 128)).shape == (128, 25)
    assert T.j_batched(m(128, 256), m(5, 128, 256), m(1, 1), m(1, 5), m(128, 1), m(1, 128)).shape == (128, 5)
    assert T.pair_energy_sym(m(256, 128), m(6, 256, 128), m(1, 1), m(1, 6), m(128, 1), m(1, 128)).shape == (128, 6)
    bf = torch.bfloat16
    assert T.ozaki_gemm(m(8, 256, 128, dt=bf), m(8, 256, 40, dt=bf)).shape == (2, 128, 40)
    assert T.ozaki_emax(m(7, 20, dt=torch.int32)).shape == (7, 1)
    assert T.ozaki_emax_col(m(7, 20, dt=torch.int32)).shape == (1, 10)
    assert T.ozaki_split(m(7, 20, dt=torch.int32), m(128, 8)).shape == (8, 128, 128)
    assert T.ozaki_split_col(m(7, 300, dt=torch.int32), m(8, 256)).shape == (8, 128, 256)
    assert T.ozaki_split(m(7, 20, dt=torch.int32), m(128, 8)).dtype == bf


def test_op_surface_dtype_checked():
    ops = d.get_native_ops()
    with pytest.raises(TypeError):
        ops["pair_energy_sym"](*(torch.zeros(2, 2, dtype=torch.float64),) * 6)
    with pytest.raises(TypeError):
        ops["gemm_ragged"](torch.zeros(2, 2, dtype=torch.int32), torch.zeros(2, 2, dtype=torch.int32))


def test_op_surface_refuses_host_tensors():
    ops = d.get_native_ops()
    with pytest.raises(Exception):
        ops["gemm_ragged"](torch.zeros(2, 2), torch.zeros(2, 2))


# ── Ozaki host half: same schedule / plan as the reference ───────────────────


@pytest.mark.parametrize("kt", [1, 3, 32, 33, 64])
@pytest.mark.parametrize("k", [1, 8, 12])
def test_schedule_matches_oracle(kt, k):
    assert ozaki.schedule(k, kt) == oracle_ozaki.schedule(k, kt)
    assert ozaki.n_groups(k, kt) == oracle_ozaki.n_groups(k, kt)


def test_k_block():
    assert ozaki.k_block(8192, 8) == 8192
    assert ozaki.k_block(4096, 12) == 4096
    for Kp, k in ((1 << 20, 8), (1 << 17, 12), (131072 + 128, 8), (1 << 18, 1)):
        kb = ozaki.k_block(Kp, k)
        assert oracle_ozaki.plan_k_blocks(Kp, k)[0][1] == kb
        assert kb % ozaki.TILE_K == 0 and kb <= Kp
    for bad in (0, 13, 2.0, True, "8"):
        with pytest.raises((ValueError, TypeError)):
            ozaki.check_slices(bad)


# ── pytorch backend (no GPU) results against the oracle ─────────────────────


def test_cpu_gemm_and_syrk_match_oracle():
    g = torch.Generator().manual_seed(0)
    A, B, C = (torch.randn(s, generator=g) for s in ((40, 30), (40, 20), (30, 20)))
    got = tb.gemm(1.0, A, B, 0.5, C, transA=True)
    assert torch.allclose(got, blas.gemm_cpu(1.0, A, B, 0.5, C, transA=True))
    S = torch.randn(40, 40, generator=g)
    got = tb.syrk(1.0, A, 0.5, S, uplo="lower")
    assert torch.allclose(got, blas.syrk_cpu(1.0, A, 0.5, S, uplo="lower"))
    assert torch.equal(got, got.T)
    Ab, Bb = torch.randn(3, 5, 7, generator=g), torch.randn(3, 7, 2, generator=g)
    assert torch.allclose(tb.batched_gemm(2.0, Ab, Bb), 2.0 * (Ab @ Bb))


def test_cpu_gemm_fp64_and_pair_energy():
    g = torch.Generator().manual_seed(1)
    A, B = torch.randn(9, 11, generator=g), torch.randn(11, 4, generator=g)
    out = tb.gemm_fp64(A, B)
    assert out.dtype == torch.float64 and torch.allclose(out, A.double() @ B.double())
    with pytest.raises(ValueError):
        tb.gemm_fp64(A, A)
    with pytest.raises(TypeError):
        tb.gemm_fp64(A.int(), B.int())
    from trnblas_amd.hip import nki_batched_pair_energy

    Bp, eo, ev = (x.float() for x in (0.05 * torch.randn(3, 8, 6, generator=g),
                                      -1 - torch.rand(3, generator=g), 1 + torch.rand(8, generator=g)))
    e = nki_batched_pair_energy(Bp, eo, ev)
    assert abs(float(e) - pe.pair_energy_f64(Bp, eo, ev)) <= 1e-5 * abs(float(e))


@pytest.mark.parametrize(
    "threads,m,n,k,want",
    [
        # measured on the MI355X box: host torch.matmul vs the upload route
        (16, 384, 384, 384, "host"),  # 0.133 ms host vs 0.169 ms upload
        (16, 512, 512, 512, "upload"),  # 0.297 vs 0.220
        (16, 16, 49152, 128, "host"),  # 0.579 vs 0.872
        (16, 128, 49152, 128, "upload"),  # 2.25 vs 1.34
        (16, 64, 4096, 4096, "upload"),  # 3.18 vs 2.81
        (2, 192, 192, 192, "host"),  # 0.076 vs 0.211
        (2, 256, 256, 256, "upload"),  # 0.152 vs 0.123
        (1, 16, 49152, 128, "upload"),  # 3.03 vs 0.872
    ],
)
def test_route_measured_crossovers(monkeypatch, threads, m, n, k, want):
    _fake_gpu(monkeypatch)
    monkeypatch.setattr(torch, "get_num_threads", lambda: threads)
    A, B = torch.empty(m, k), torch.empty(k, n)
    assert d._gemm_route(A, B) == want


def test_pair_energy_math_selection(monkeypatch):
    from trnblas_amd.hip import kernels

    monkeypatch.delenv("TRNBLAS_PAIR_ENERGY_MATH", raising=False)
    assert kernels.pair_energy_math() == "fp16x3"
    monkeypatch.setenv("TRNBLAS_PAIR_ENERGY_MATH", "fp32")
    assert kernels.pair_energy_math() == "fp32"
    assert kernels._check_math(None) == "fp32"
    assert kernels._check_math("bf16x6") == "bf16x6"
    monkeypatch.setenv("TRNBLAS_PAIR_ENERGY_MATH", "tf32")
    with pytest.raises(ValueError):
        kernels.pair_energy_math()
    assert kernels._PE_ENTRY["bf16x6"] == "trnblas_hip_pair_energy_bf16x6"
    assert kernels._PE_ENTRY["fp16x3"] == "trnblas_hip_pair_energy_fp16x3"
    assert kernels._check_math("fp16x3") == "fp16x3"


# ── autotune (measured kernel-vs-hipBLASLt route, cached per shape bucket) ───


def test_autotune_bucket_key():
    from trnblas_amd.hip import dispatch as d

    k = d._autotune_key((1000, 300), (300, 70), torch.bfloat16, False, False, True)
    assert k == "bfloat16,001,1,1024,512,128"  # power-of-two ceilings of batch, M, K, N
    # shapes within one bucket share the key, the next power of two does not
    assert d._autotune_key((600, 257), (257, 65), torch.bfloat16, False, False, True) == k
    assert d._autotune_key((1025, 300), (300, 70), torch.bfloat16, False, False, True) != k
    # batch broadcast, layout and dtype are part of the key
    kb = d._autotune_key((3, 1, 64, 64), (5, 64, 64), torch.float16, False, True, False)
    assert kb == "float16,010,16,64,64,64"


def test_autotune_cache_round_trip(monkeypatch, tmp_path):
    from trnblas_amd.hip import dispatch as d

    path = tmp_path / "sub" / "cache.json"
    monkeypatch.setattr(d, "_AUTOTUNE_CACHE_FILE", str(path))
    monkeypatch.setattr(d, "_autotune_mem", {"bfloat16,001,1,1024,512,128": "aten"})
    monkeypatch.setattr(d, "_autotune_loaded", True)
    d._save_autotune_cache()  # creates the directory
    monkeypatch.setattr(d, "_autotune_mem", {})
    monkeypatch.setattr(d, "_autotune_loaded", False)
    d._load_autotune_cache()
    assert d._autotune_mem == {"bfloat16,001,1,1024,512,128": "aten"}
    # unknown route names and unreadable files are ignored
    path.write_text('{"a": "hip", "b": "cuda"}')
    monkeypatch.setattr(d, "_autotune_loaded", False)
    d._load_autotune_cache()
    assert d._autotune_mem == {"a": "hip"}
    path.write_text("not json")
    monkeypatch.setattr(d, "_autotune_loaded", False)
    d._load_autotune_cache()
    assert d._autotune_mem == {}


def test_autotune_flag_and_inadmissible_operands(monkeypatch):
    from trnblas_amd.hip import dispatch as d

    monkeypatch.setattr(d, "_AUTOTUNE", False)
    tb.set_autotune(True)
    assert tb.get_autotune() is True
    tb.set_autotune(False)
    assert tb.get_autotune() is False
    # fp32, SYRK and mixed-rank operands are never timed: the static rule decides
    a = torch.empty(64, 64)
    assert d._autotune_gemm_route(a, a, "gemm") is None
    h = a.bfloat16()
    assert d._autotune_gemm_route(h, h, "syrk") is None
    assert d._autotune_gemm_route(h.expand(2, 64, 64), h, "batched_gemm") is None


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,N,K,shift", [(37, 53, 71, False), (16, 24, 32, True), (5, 8, 3, False), (64, 64, 64, False)])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_packed_operands_are_dma_ready_and_exact(monkeypatch, dtype, M, N, K, shift, ta, tb):
    # the host side of operand packing, on CPU tensors: the C-ABI arguments
    # it returns describe 16-byte-ready operands (every check the library's
    # DMA gate makes) which, read as the kernel reads them, are the original
    # operands with zero columns of A and zero rows of B appended along K
    from trnblas_amd.hip import kernels as k

    monkeypatch.setattr(k, "PACK_MIN_MACS", {4: 0, 2: 0})

    def pack_on_host(X, kp):  # trnblas_hip_pack_k's result, for CPU tensors
        P = torch.zeros((*X.shape[:-1], kp), dtype=X.dtype)
        P[..., : X.shape[-1]] = X
        return P

    monkeypatch.setattr(k, "_pack_k", pack_on_host)
    g = torch.Generator().manual_seed(M + N + K + 2 * ta + tb)
    A = torch.randn(K, M, generator=g).T if ta else torch.randn(M, K, generator=g)
    B = torch.randn(N, K, generator=g).T if tb else torch.randn(K, N, generator=g)
    A, B = A.to(dtype), B.to(dtype)
    if shift:
        buf = torch.empty(A.numel() + 1, dtype=dtype)
        A = buf[1:].view(M, K).copy_(A)
    a, ta2, lda = k._mat_layout(A)
    b, tb2, ldb = k._mat_layout(B)
    a, ta2, lda, _, b, tb2, ldb, _, kp = k._packed_operands(A, B, a, ta2, lda, 0, b, tb2, ldb, 0, M, N, K, 1)
    ev = 16 // A.element_size()
    assert kp % ev == 0 and kp >= K
    assert k._dma_ready(a, lda, 0, M if ta2 else kp, ev) and k._dma_ready(b, ldb, 0, kp if tb2 else N, ev)
    A2 = torch.as_strided(a, (M, kp), (1, lda) if ta2 else (lda, 1))
    B2 = torch.as_strided(b, (kp, N), (1, ldb) if tb2 else (ldb, 1))
    assert torch.equal(A2[:, :K], A) and torch.equal(B2[:K], B)
    assert not A2[:, K:].any() and not B2[K:].any()
    if not (K % ev or shift or (ta and M % ev) or (not tb and N % ev)):
        assert a is A or a.data_ptr() == A.data_ptr()  # ready operands are not copied


def test_packed_operands_below_threshold_untouched():
    from trnblas_amd.hip import kernels as k

    A, B = torch.randn(37, 71), torch.randn(71, 53)
    out = k._packed_operands(A, B, A, False, 71, 0, B, False, 53, 0, 37, 53, 71, 1)
    assert out[0] is A and out[4] is B and out[8] == 71


def test_unready_16bit_route_rule():
    # 16-bit 2-D operands the DMA kernel cannot read in place go to hipBLASLt
    # from 2^26 multiply-adds (stride logic only, on CPU tensors)
    bf = torch.bfloat16
    A, B = torch.zeros(512, 512, dtype=bf), torch.zeros(512, 512, dtype=bf)
    assert not d._unready_16bit_to_aten(A, B, "gemm")  # ready
    A3, B3 = torch.zeros(511, 511, dtype=bf), torch.zeros(511, 511, dtype=bf)
    assert d._unready_16bit_to_aten(A3, B3, "gemm")  # ragged K / N
    assert d._unready_16bit_to_aten(A3.T, B3.T, "gemm")  # transposed views, ragged M / K
    assert not d._unready_16bit_to_aten(A3, B3, "syrk")
    assert not d._unready_16bit_to_aten(A3.float(), B3.float(), "gemm")  # fp32 stays
    small = torch.zeros(255, 255, dtype=bf)
    assert not d._unready_16bit_to_aten(small, small, "gemm")  # below 2^26
    buf = torch.zeros(512 * 512 + 1, dtype=bf)
    off = buf[1:].view(512, 512)  # one element off a 16-byte boundary
    assert d._unready_16bit_to_aten(off, B, "gemm")
    assert d._dma_ready_2d(torch.zeros(64, 64, dtype=bf).T, 64, 64)


# ── drop-in switches read from the environment ──────────────────────────────


@pytest.mark.parametrize("value,on", [(None, True), ("1", True), ("yes", True), ("0", False),
                                      ("false", False), (" Off ", False), ("no", False)])
def test_pinned_output_switch(monkeypatch, value, on):
    # TRNBLAS_PINNED_OUTPUT (nki/dispatch.py:2052-2060), read at every call
    if value is None:
        monkeypatch.delenv("TRNBLAS_PINNED_OUTPUT", raising=False)
    else:
        monkeypatch.setenv("TRNBLAS_PINNED_OUTPUT", value)
    assert d._pinned_output_enabled() is on
    t = torch.arange(6.0)
    assert d._to_host(t, torch.device("cpu")) is t  # host tensors are never copied


def test_metric_solve_switch(monkeypatch):
    # TRNBLAS_METRIC_SOLVE=auto|host|device (nki/dispatch.py:1833-1849)
    J = torch.eye(4, dtype=torch.float64) * 4.0
    for v in ("auto", "host", "device", " HOST "):
        monkeypatch.setenv("TRNBLAS_METRIC_SOLVE", v)
        assert d._metric_solve_route(J) == "device"  # a host J: host LAPACK through torch
        assert torch.allclose(d.nki_metric_inv_half(J), torch.eye(4, dtype=torch.float64) * 0.5)
    monkeypatch.setenv("TRNBLAS_METRIC_SOLVE", "gpu")
    with pytest.raises(ValueError, match="TRNBLAS_METRIC_SOLVE"):
        d.nki_metric_inv_half(J)


def test_ozaki_device_split_switch_warns_once(monkeypatch):
    # TRNBLAS_OZAKI_DEVICE_SPLIT=0 (nki/dispatch.py:853-862) cannot change the
    # digits here (the split is native fp64 on the device): one warning says so
    monkeypatch.setattr(d, "_oz_split_noted", False)
    monkeypatch.setenv("TRNBLAS_OZAKI_DEVICE_SPLIT", "0")
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        d._note_ozaki_device_split()
        d._note_ozaki_device_split()
    assert len([x for x in w if "TRNBLAS_OZAKI_DEVICE_SPLIT" in str(x.message)]) == 1
    monkeypatch.setattr(d, "_oz_split_noted", False)
    monkeypatch.setenv("TRNBLAS_OZAKI_DEVICE_SPLIT", "1")
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        d._note_ozaki_device_split()
    assert not w


def test_gemm_ragged_switch(monkeypatch):
    # TRNBLAS_GEMM_RAGGED=0 (nki/dispatch.py:144-151): operands the DMA kernel
    # cannot read are packed and zero-padded at every size
    from trnblas_amd.hip import kernels as k

    monkeypatch.setattr(k, "_pack_k", lambda X, kp: torch.nn.functional.pad(X, (0, kp - X.shape[-1])))
    A, B = torch.randn(37, 71), torch.randn(71, 53)
    args = (A, B, A, False, 71, 0, B, False, 53, 0, 37, 53, 71, 1)
    assert k._packed_operands(*args)[8] == 71  # on: small products stay in place
    monkeypatch.setattr(k, "_RAGGED_ENABLED", False)
    out = k._packed_operands(*args)
    assert out[8] == 72 and out[0] is not A and torch.equal(out[0][:, :71], A)
    code = "import trnblas_amd.hip.kernels as k; print(k._RAGGED_ENABLED)"
    for v, want in (("0", "False"), ("off", "False"), ("1", "True")):
        env = dict(__import__("os").environ, TRNBLAS_GEMM_RAGGED=v)
        r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env)
        assert r.stdout.strip() == want, (v, r.stderr)


def test_autotune_skips_capture_and_survives_hipblaslt_failure(monkeypatch, tmp_path):
    # no timing inside a graph capture; a hipBLASLt failure keeps the kernel
    from trnblas_amd.hip import dispatch as d
    from trnblas_amd.hip import kernels as k

    monkeypatch.setattr(d, "_autotune_mem", {})
    monkeypatch.setattr(d, "_autotune_loaded", True, raising=False)
    monkeypatch.setattr(d, "_save_autotune_cache", lambda: None)
    h = torch.empty(64, 64, dtype=torch.bfloat16)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    monkeypatch.setattr(d, "_time_device_call", lambda f: pytest.fail("timed during capture"))
    assert d._autotune_gemm_route(h, h, "gemm") is None
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    calls = []

    def timed(f):
        calls.append(f)
        if len(calls) == 2:
            raise RuntimeError("hipBLASLt failed")
        return 1.0

    monkeypatch.setattr(d, "_time_device_call", timed)
    monkeypatch.setattr(k, "gemm", lambda a, b: None)
    assert d._autotune_gemm_route(h, h, "gemm") == "hip"
    assert len(calls) == 2 and not d._autotune_mem  # not cached


@pytest.mark.parametrize("Mp,Kp,N,k,limit", [
    (4096, 4096, 4096, 8, ozaki.BLOCK_BYTES), (16384, 16384, 241, 8, ozaki.BLOCK_BYTES),
    (3328, 8448, 241, 8, ozaki.BLOCK_BYTES), (1024, 2048, 3000, 8, 1 << 22), (256, 1 << 20, 64, 10, 1 << 26),
])  # fmt: skip
def test_ozaki_plan_interface(Mp, Kp, N, k, limit):
    # the reference's launch-plan contract (tests/test_ozaki.py:145-166)
    mbs, kbs, nbs = ozaki.plan(Mp, Kp, N, k, limit)
    for blocks, D in ((mbs, Mp), (kbs, Kp), (nbs, N)):
        assert blocks[0][0] == 0 and sum(sz for _, sz in blocks) == D
        assert all(a + sa == b for (a, sa), (b, _) in zip(blocks, blocks[1:]))
    assert all(sz % 128 == 0 for _, sz in mbs + kbs)
    Mb, Kb, Nb = mbs[0][1], kbs[0][1], nbs[0][1]
    assert 2 * k * Kb * Mb <= limit and 2 * k * Kb * Nb <= limit and 8 * Mb * Nb <= limit
    assert Mb <= ozaki.LAUNCH_M and Nb <= ozaki.LAUNCH_N
    assert Kb == ozaki.k_block(Kp, k, limit)
    if limit == ozaki.BLOCK_BYTES and Mp * Kp * 2 * k <= limit:
        assert len(kbs) == 1


def test_ozaki_plan_known_answers():
    assert len(ozaki.plan(768, 1024, 600, 4, max_m=256, max_n=200)[0]) == 3
    mbs, kbs, nbs = ozaki.plan(2304, 512, 1500, 3, 2 * 3 * 512 * 1024)
    assert len(mbs) > 1 and len(nbs) > 1 and len(kbs) == 1
    assert len(ozaki.plan(128, 3072, 20, 8, 2 * 8 * 128 * 1024)[1]) > 1
