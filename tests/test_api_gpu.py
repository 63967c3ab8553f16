"""GPU parity of the public API (trnblas_amd.gemm / batched_gemm / syrk /
gemm_fp64 / nki_batched_pair_energy) at the BASELINE configurations and at
edge cases, against the oracle (the reference's CPU path restated) and
fp64 closed forms. Every call goes through the C ABI (TRNBLAS_REQUIRE_HIP
makes a kernel error raise instead of falling back)."""

import os

import numpy as np
import pytest
import torch

import trnblas_amd as tb
from oracle import blas, exact
from oracle import ozaki as oz
from oracle import pair_energy as pe
from trnblas_amd import df_mp2

pytestmark = pytest.mark.gpu


def _cw(D, ref, den):
    den = torch.where(den > 0, den, torch.ones_like(den))
    return float(((D.double() - ref) / den).abs().max())


# ── C1: gemm fp32, transA, alpha 1, beta 0.5, 2048^3 ────────────────────────


def test_config1_gemm_matches_cpu_path(dev):
    A, B, C = df_mp2.config1_inputs(dev)
    Cin = C.clone()
    D = tb.gemm(1.0, A, B, beta=0.5, C=C, transA=True)
    torch.cuda.synchronize()
    assert torch.equal(C, Cin)  # C never written
    Ah, Bh, Ch = A.cpu(), B.cpu(), C.cpu()
    cpu = blas.gemm_cpu(1.0, Ah, Bh, 0.5, Ch, transA=True)  # the reference's CPU path
    ref = blas.gemm_f64(1.0, Ah, Bh, 0.5, Ch, transA=True)
    den = blas.gemm_cw_den(1.0, Ah, Bh, 0.5, Ch, transA=True)
    assert _cw(D.cpu(), cpu.double(), den) <= 1e-6  # north-star gate vs the CPU path
    assert _cw(D.cpu(), ref, den) <= 1e-6


# ── C2: SYRK 4096 x 8192 lower + batched 64 x 512 x 2048 x 512 ───────────────


def test_config2_syrk_and_batched(dev):
    A, C, Ab, Bb = df_mp2.config2_inputs(dev)
    S = tb.syrk(1.0, A, beta=0.5, C=C, uplo="lower")
    Db = tb.batched_gemm(1.0, Ab, Bb)
    torch.cuda.synchronize()
    assert torch.equal(S, S.T)
    Ad = A.double()
    ref = Ad @ Ad.T + 0.5 * (torch.tril(C.double()) + torch.tril(C.double(), -1).T)
    den = Ad.abs() @ Ad.abs().T + 0.5 * C.double().abs()
    assert _cw(S, ref, den) <= 1e-6  # north-star gate vs fp64
    # ... and vs the reference's CPU path (fp32 torch.matmul + the epilogue)
    Sh = S.cpu()
    cpu = blas.syrk_cpu(1.0, A.cpu(), 0.5, C.cpu(), uplo="lower")
    assert _cw(Sh, cpu.double(), den.cpu()) <= 1e-6
    refb = Ab.double() @ Bb.double()
    denb = Ab.double().abs() @ Bb.double().abs()
    assert _cw(Db, refb, denb) <= 1e-6
    cpub = blas.gemm_cpu(1.0, Ab.cpu(), Bb.cpu())
    assert _cw(Db.cpu(), cpub.double(), denb.cpu()) <= 1e-6


def test_gemm_same_sign_long_k(dev):
    # U(0, 1) operands: every output is a sum of K same-sign products, the
    # case in which the rounding of one long fp32 accumulation chain adds up
    # (cancelling N(0, 1) data hides it). Gate: 1e-6 |A||B| against fp64 and
    # against the reference's CPU path.
    g = torch.Generator().manual_seed(11)
    K = 8192
    A = torch.rand(1024, K, generator=g)
    B = torch.rand(K, 768, generator=g)
    C = torch.rand(1024, 768, generator=g)
    D = tb.gemm(1.0, A.to(dev), B.to(dev), beta=0.5, C=C.to(dev)).cpu()
    ref = blas.gemm_f64(1.0, A, B, 0.5, C)
    den = blas.gemm_cw_den(1.0, A, B, 0.5, C)
    assert _cw(D, ref, den) <= 1e-6
    cpu = blas.gemm_cpu(1.0, A, B, 0.5, C)
    assert _cw(D, cpu.double(), den) <= 1e-6
    # transposed read paths (C1's layout) and SYRK on the same data
    Dt = tb.gemm(1.0, A.T.contiguous().to(dev), B.to(dev), transA=True).cpu()
    assert _cw(Dt, A.double() @ B.double(), A.double() @ B.double()) <= 1e-6
    S = tb.syrk(1.0, A[:640].to(dev), uplo="lower").cpu()
    As = A[:640].double()
    assert _cw(S, As @ As.T, As @ As.T) <= 1e-6


@pytest.mark.parametrize("n,k", [(1030, 260), (1030, 1000), (1024, 2500), (768, 4096)])
@pytest.mark.parametrize("trans", [False, True])
def test_syrk_same_sign_short_k(dev, n, k, trans):
    # U(0, 1) operands with K of a few hundred to a few thousand: one
    # accumulation chain carries most of each sum (with 256-long chains the
    # largest error over a 1030^2 SYRK at K = 260 was 1.05e-6). Gate: 1e-6
    # against fp64 and against the reference's CPU path; the output covers
    # ~1M elements, so the gate holds at the tail, not only on average.
    g = torch.Generator().manual_seed(n + k + int(trans))
    A = torch.rand((k, n) if trans else (n, k), generator=g)
    S = tb.syrk(1.0, A.to(dev), trans=trans, uplo="lower").cpu()
    op = (A.T if trans else A).double()
    ref, den = op @ op.T, op @ op.T
    assert _cw(S, ref, den) <= 1e-6
    cpu = blas.syrk_cpu(1.0, A, trans=trans, uplo="lower").double()
    # the CPU path's own error against fp64 (its transposed reads can be
    # less accurate than the gate) bounds how far the two may differ
    assert _cw(S, cpu, den) <= 1e-6 + _cw(cpu.float(), ref, den)
    G = tb.gemm(1.0, op.float().to(dev), op.T.contiguous().float().to(dev)).cpu()
    assert _cw(G, ref, den) <= 1e-6


# ── GEMM semantics and edge cases ────────────────────────────────────────────


def test_gemm_edge_cases(dev):
    g = torch.Generator(device=dev).manual_seed(0)
    A = torch.randn(70, 50, device=dev, generator=g)
    B = torch.randn(50, 30, device=dev, generator=g)
    Cnan = torch.full((70, 30), float("nan"), device=dev)
    assert torch.isfinite(tb.gemm(1.0, A, B, beta=0.0, C=Cnan)).all()  # beta 0: C not read
    row = torch.randn(30, device=dev, generator=g)
    out = tb.gemm(2.0, A, B, beta=-1.0, C=row)  # broadcast C
    assert torch.allclose(out, 2.0 * (A @ B) - row, atol=1e-4)
    assert tb.gemm(1.0, A[:0], B).shape == (0, 30)
    z = tb.gemm(1.0, A[:, :0], B[:0], beta=0.5, C=torch.ones(70, 30, device=dev))
    assert torch.equal(z, torch.full((70, 30), 0.5, device=dev))  # K = 0
    # bf16 and transposed views
    Ab, Bb = A.bfloat16(), B.bfloat16()
    out = tb.gemm(1.0, Ab.T.contiguous(), Bb, transA=True)
    assert out.dtype == torch.bfloat16
    assert torch.allclose(out.float(), Ab.float() @ Bb.float(), rtol=2e-2, atol=0.2)
    # a C of another dtype: torch promotion semantics
    out = tb.gemm(1.0, A, B, beta=1.0, C=torch.ones(70, 30, device=dev, dtype=torch.float64))
    assert out.dtype == torch.float64


def test_batched_gemm_broadcast_and_4d(dev):
    g = torch.Generator(device=dev).manual_seed(1)
    A = torch.randn(2, 3, 20, 10, device=dev, generator=g)
    B = torch.randn(10, 7, device=dev, generator=g)
    C = torch.randn(20, 7, device=dev, generator=g)
    out = tb.batched_gemm(1.0, A, B, beta=0.5, C=C)
    assert out.shape == (2, 3, 20, 7)
    assert torch.allclose(out, A @ B + 0.5 * C, atol=1e-4)
    A3 = torch.randn(5, 10, 20, device=dev, generator=g)
    out = tb.batched_gemm(1.0, A3, B.T.contiguous().expand(5, 7, 10), transA=True, transB=True)
    assert torch.allclose(out, A3.transpose(1, 2) @ B, atol=1e-4)


def test_syrk_variants(dev):
    g = torch.Generator(device=dev).manual_seed(2)
    A = torch.randn(300, 77, device=dev, generator=g)
    X = torch.randn(300, 300, device=dev, generator=g)
    for trans, uplo in [(False, "upper"), (True, "lower")]:
        a = A.T.contiguous() if trans else A
        out = tb.syrk(1.5, a, beta=-0.5, C=X, trans=trans, uplo=uplo)
        assert torch.equal(out, out.T)
        ref = blas.syrk_f64(1.5, a.cpu(), -0.5, X.cpu(), trans=trans, uplo=uplo)
        assert (out.cpu().double() - ref).abs().max() < 1e-3
    with pytest.warns(DeprecationWarning):
        out = tb.syrk(1.0, A, beta=1.0, C=torch.tril(X), uplo="upper")
    ref = blas.syrk_f64(1.0, A.cpu(), 1.0, torch.tril(X).cpu(), uplo="lower")
    assert (out.cpu().double() - ref).abs().max() < 1e-3
    out = tb.syrk(2.0, A)  # no C
    assert torch.equal(out, out.T)


# ── C3: fused DF-MP2 pair energy 96 / 672 / 2304 ─────────────────────────────


def _pair_energy_f64_gpu(B, eo, ev):
    """The fp64 closed form on the GPU (symmetric walk, fp64 GEMMs)."""
    Bd, eod, evd = B.double(), eo.double(), ev.double()
    nocc = B.shape[0]
    tot = torch.zeros((), dtype=torch.float64, device=B.device)
    for i in range(nocc):
        T = torch.matmul(Bd[i].unsqueeze(0), Bd[i:].transpose(1, 2))
        D = eod[i] + eod[i:, None, None] - evd[None, :, None] - evd[None, None, :]
        e = (T * (2.0 * T - T.transpose(1, 2)) / D).sum(dim=(1, 2))
        w = torch.full_like(e, 2.0)
        w[0] = 1.0
        tot += (w * e).sum()
    return float(tot)


def test_config3_pair_energy_fp64_gate(dev):
    from trnblas_amd.hip import nki_batched_pair_energy

    B, eo, ev = df_mp2.config3_inputs(dev)
    e = nki_batched_pair_energy(B, eo, ev)
    assert e.dtype == torch.float32 and e.dim() == 0
    got = float(tb.hip.kernels.pair_energy_sym(B, eo, ev))  # fp64 total
    want = _pair_energy_f64_gpu(B, eo, ev)
    assert abs(got - want) <= 1e-6 * abs(want), (got, want)
    assert abs(float(e) - want) <= 1e-6 * abs(want)


@pytest.mark.parametrize("shape", [(5, 97, 130), (16, 128, 384), (1, 672, 2304), (3, 1000, 33)])
def test_pair_energy_shapes_vs_oracle(dev, shape):
    from trnblas_amd.hip import nki_batched_pair_energy

    B, eo, ev = df_mp2.pair_inputs(*shape, seed=sum(shape))
    got = float(tb.hip.kernels.pair_energy_sym(B.to(dev), eo.to(dev), ev.to(dev)))
    want = pe.pair_energy_f64(B, eo, ev)
    assert abs(got - want) <= 1e-6 * abs(want)
    assert abs(float(nki_batched_pair_energy(B, eo, ev)) - want) <= 1e-6 * abs(want)  # host in


def test_energy_reduction_paths_agree(dev):
    B, eo, ev = df_mp2.pair_inputs(6, 100, 64, dev, seed=5)
    want = pe.pair_energy_f64(B, eo, ev)
    assert abs(df_mp2.energy_reduction(B, eo, ev) - want) <= 1e-5 * abs(want)
    assert abs(df_mp2.energy_reduction_batched_pair(B, eo, ev) - want) <= 1e-6 * abs(want)


def test_energy_legacy_entry_points(dev):
    from trnblas_amd.hip import nki_fused_gemm_energy, nki_mp2_energy

    B, eo, ev = df_mp2.pair_inputs(4, 60, 48, dev, seed=6)
    e = nki_fused_gemm_energy(B[1], B[3], float(eo[1]), float(eo[3]), ev)
    want = float(pe.fused_pair_cpu(B[1].double().cpu(), B[3].double().cpu(), float(eo[1]), float(eo[3]), ev.double().cpu()))
    assert abs(float(e) - want) <= 1e-6 * abs(want)
    flat = B.reshape(4 * 60, 48)
    T_flat = flat[:120] @ flat.T
    e = nki_mp2_energy(T_flat, eo[:2], eo, ev)
    want = float(pe.mp2_energy_cpu(T_flat.double().cpu(), eo[:2].double().cpu(), eo.double().cpu(), ev.double().cpu()))
    assert abs(float(e) - want) <= 1e-6 * abs(want)


def test_config4_chain_small(dev):
    eri, Co, Cv, eo, ev = df_mp2.chain_inputs(64, 8, 24, 96, dev, seed=4)
    B = df_mp2.half_transform(eri, Co, Cv)
    ref = torch.einsum("mi,na,pmn->iap", Co.double(), Cv.double(), eri.double())
    assert B.shape == (8, 24, 96)
    assert (B.double() - ref).abs().max() <= 1e-5 * ref.abs().max()
    e = df_mp2.df_mp2_chain_energy(eri, Co, Cv, eo, ev)
    want = pe.pair_energy_f64(ref.cpu(), eo.cpu(), ev.cpu())
    assert abs(e - want) <= 1e-5 * abs(want)


# ── C5: Ozaki gemm_fp64 ──────────────────────────────────────────────────────


@pytest.mark.parametrize(
    "M,K,N,k,views",
    [(37, 300, 53, 7, ""), (130, 4100, 7, 8, ""), (200, 600, 520, 8, "AB"), (5, 4100, 3, 8, "A"),
     (64, 64, 64, 12, "B"), (1, 1, 1, 8, ""), (600, 700, 650, 8, ""), (6, 90000, 3, 12, "")],
)
def test_gemm_fp64_bitwise_vs_reference(dev, M, K, N, k, views):
    A, B = exact.inputs(M, K, N, seed=M * 3 + N)
    Ad = torch.from_numpy(A).to(dev)
    Bd = torch.from_numpy(B).to(dev)
    if "A" in views:  # transposed-view operand, read in place
        Ad = torch.from_numpy(np.ascontiguousarray(A.T)).to(dev).T
    if "B" in views:
        Bd = torch.from_numpy(np.ascontiguousarray(B.T)).to(dev).T
    C = tb.gemm_fp64(Ad, Bd, slices=k, mode="exact")
    assert C.dtype == torch.float64 and C.device == Ad.device
    want = oz.reference_gemm(A, B, k)
    assert np.array_equal(C.cpu().numpy().view(np.int64), want.view(np.int64))


def test_gemm_fp64_golden_from_reference(dev):
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "ozaki_golden.npz"))
    for c in range(5):
        A, B, Cw = gold[f"gemm{c}_A"], gold[f"gemm{c}_B"], gold[f"gemm{c}_C"]
        C = tb.gemm_fp64(
            torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev), slices=int(gold[f"gemm{c}_k"]),
            mode="exact",
        )
        assert np.array_equal(C.cpu().numpy().view(np.int64), Cw.view(np.int64)), c


@pytest.mark.parametrize(
    "M,K,N,k,dist,views",
    [(37, 300, 53, 7, "normal", ""), (130, 4100, 7, 8, "normal", ""), (200, 600, 520, 8, "logu4", "AB"),
     (5, 4100, 3, 8, "normal", "A"), (64, 64, 64, 12, "normal", "B"), (1, 1, 1, 8, "normal", ""),
     (70, 257, 90, 1, "normal", ""), (66, 1000, 130, 3, "logu4", ""), (129, 384, 65, 10, "logu4", "")],
)
def test_gemm_fp64_fast_within_bound(dev, M, K, N, k, dist, views):
    # fast mode: every element within the k-slice truncation bound of the
    # exact (rational) product, and no further from it than the exact mode's
    # fp32 (hi, lo) floor
    A, B = exact.inputs(M, K, N, dist=dist, seed=M * 5 + N + k)
    Ad = torch.from_numpy(A).to(dev)
    Bd = torch.from_numpy(B).to(dev)
    if "A" in views:
        Ad = torch.from_numpy(np.ascontiguousarray(A.T)).to(dev).T
    if "B" in views:
        Bd = torch.from_numpy(np.ascontiguousarray(B.T)).to(dev).T
    C = tb.gemm_fp64(Ad, Bd, slices=k, mode="fast").cpu().numpy()
    ref = exact.ref_exact(A, B)
    bound = oz.error_bound(A, B, k)
    assert (np.abs(C - ref) <= bound).all()
    Cx = oz.reference_gemm(A, B, k)
    AB = np.abs(A) @ np.abs(B)
    assert (np.abs(C - Cx) <= 2.0**-45 * AB + 1e-300).all()


def test_gemm_fp64_fast_flush_path(dev):
    # k = 12 and K = 44032: k * K * 2^12 passes 2^31, so the int32 diagonals
    # are flushed to fp64 once mid-K (the block path that adds into C)
    A, B = exact.inputs(40, 44032, 24, seed=77)
    C = tb.gemm_fp64(torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev), slices=12, mode="fast")
    C = C.cpu().numpy()
    ref = exact.ref_exact(A, B)
    assert (np.abs(C - ref) <= oz.error_bound(A, B, 12)).all()
    err = float((np.abs(C - ref) / (np.abs(A) @ np.abs(B))).max())
    assert err <= 1e-15, err


def test_gemm_fp64_nonfinite_and_empty(dev):
    A = torch.randn(20, 30, dtype=torch.float64, device=dev)
    B = torch.randn(30, 10, dtype=torch.float64, device=dev)
    A[3, 4] = float("inf")
    C = tb.gemm_fp64(A, B)
    assert torch.equal(C.isinf(), (A @ B).isinf()) and torch.equal(C.isnan(), (A @ B).isnan())
    assert tb.gemm_fp64(A[:, :0], B[:0]).abs().sum() == 0
    assert tb.gemm_fp64(A[:0], B).shape == (0, 10)


def test_config5_gemm_fp64_accuracy_full_size(dev):
    # C5 at 8192^3 on its wide-range data: every element within the
    # reference's k-slice error bound (oracle.ozaki.error_bound: the
    # per-row / per-column truncation of ozaki.py:123-139 plus the
    # double-fp32 floor), against native fp64 DGEMM.
    n = 8192
    A, B = df_mp2.config5_inputs(dev, n, seed=5)
    g = torch.Generator(device=dev).manual_seed(6)
    ref = A @ B
    AB = A.abs() @ B.abs()
    bound = oz.error_bound(A, B, 8, absA_absB=AB, xp=torch) + n * 2.0**-53 * AB
    for mode in ("fast", "exact"):
        C = tb.gemm_fp64(A, B, mode=mode)
        assert bool(((C - ref).abs() <= bound).all()), mode
        del C
    # on well-scaled data k = 8 is host-fp64 accurate (test_ozaki.py:179-187)
    A2 = torch.randn(4096, 4096, generator=g, device=dev, dtype=torch.float64)
    B2 = torch.randn(4096, 4096, generator=g, device=dev, dtype=torch.float64)
    for mode in ("fast", "exact"):
        C2 = tb.gemm_fp64(A2, B2, mode=mode)
        err = float(((C2 - A2 @ B2).abs() / (A2.abs() @ B2.abs())).max())
        assert err <= 1.5e-15, (mode, err)
