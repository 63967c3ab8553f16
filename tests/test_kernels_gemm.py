"""GPU parity of the HIP GEMM / SYRK kernels against an fp64 torch reference
(the componentwise gate of trnblas's north star: |C - C_ref| <= 1e-6 (|A||B|)ij
for fp32), through the C ABI (trnblas_amd.hip.kernels)."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _ref(A, B, alpha, beta, C):
    R = alpha * (A.double() @ B.double())
    if C is not None and beta != 0:
        R = R + beta * C.double()
    return R


def _cw_err(D, A, B, alpha, beta, C):
    den = abs(alpha) * (A.double().abs() @ B.double().abs())
    if C is not None and beta != 0:
        den = den + abs(beta) * C.double().abs()
    den = torch.where(den > 0, den, torch.ones_like(den))
    return ((D.double() - _ref(A, B, alpha, beta, C)).abs() / den).max().item()


@pytest.mark.parametrize(
    "M,N,K",
    [(128, 128, 16), (256, 384, 512), (1, 1, 1), (37, 53, 71), (130, 257, 1000), (64, 200, 3)],
)
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_gemm_fp32_layouts(dev, M, N, K, ta, tb):
    from trnblas_amd.hip import kernels

    g = torch.Generator().manual_seed(M * 7 + N * 3 + K)
    A0 = torch.randn((K, M) if ta else (M, K), generator=g)
    B0 = torch.randn((N, K) if tb else (K, N), generator=g)
    C = torch.randn(M, N, generator=g)
    A = (A0.mT if ta else A0).to(dev)
    B = (B0.mT if tb else B0).to(dev)
    D = kernels.gemm(A, B, 1.0, 0.5, C.to(dev))
    torch.cuda.synchronize()
    err = _cw_err(D.cpu(), A.cpu(), B.cpu(), 1.0, 0.5, C)
    assert err <= 1e-6, err


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 2e-2), (torch.float16, 3e-3)])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_gemm_16bit(dev, dtype, tol, ta, tb):
    from trnblas_amd.hip import kernels

    M, N, K = 200, 136, 300
    g = torch.Generator().manual_seed(1)
    A0 = torch.randn((K, M) if ta else (M, K), generator=g).to(dtype)
    B0 = torch.randn((N, K) if tb else (K, N), generator=g).to(dtype)
    A = (A0.mT if ta else A0).to(dev)
    B = (B0.mT if tb else B0).to(dev)
    D = kernels.gemm(A, B, 2.0)
    torch.cuda.synchronize()
    assert D.dtype == dtype
    ref = 2.0 * (A.cpu().double() @ B.cpu().double())
    den = 2.0 * (A.cpu().double().abs() @ B.cpu().double().abs())
    assert ((D.cpu().double() - ref).abs() / den).max().item() <= tol


def test_gemm_batched_broadcast(dev):
    from trnblas_amd.hip import kernels

    g = torch.Generator().manual_seed(2)
    A = torch.randn(5, 70, 90, generator=g)
    B = torch.randn(1, 90, 33, generator=g)
    C = torch.randn(70, 33, generator=g)
    D = kernels.gemm(A.to(dev), B.to(dev), 1.5, -0.25, C.to(dev))
    torch.cuda.synchronize()
    ref = 1.5 * (A.double() @ B.double()) - 0.25 * C.double()
    assert (D.cpu().double() - ref).abs().max().item() < 1e-3


@pytest.mark.parametrize("n,k", [(256, 128), (300, 77), (1, 5), (129, 1000)])
@pytest.mark.parametrize("trans", [False, True])
@pytest.mark.parametrize("uplo", ["lower", "upper"])
def test_syrk_triangle(dev, n, k, trans, uplo):
    from trnblas_amd.hip import kernels

    g = torch.Generator().manual_seed(n + k)
    A = torch.randn((k, n) if trans else (n, k), generator=g)
    X = torch.randn(n, n, generator=g)
    D = kernels.syrk(A.to(dev), 1.0, 0.5, X.to(dev), trans=trans, uplo=uplo)
    torch.cuda.synchronize()
    D = D.cpu()
    assert torch.equal(D, D.T)
    opA = A.T if trans else A
    Cs = torch.tril(X) + torch.tril(X, -1).T if uplo == "lower" else torch.triu(X) + torch.triu(X, 1).T
    ref = opA.double() @ opA.double().T + 0.5 * Cs.double()
    den = opA.double().abs() @ opA.double().abs().T + 0.5 * Cs.double().abs()
    # SYRK diagonals are sums of k positive terms: the same 1e-6 gate
    assert ((D.double() - ref).abs() / den).max().item() <= 1e-6


@pytest.mark.parametrize(
    "M,N,K,ta,tb",
    [(1024, 1024, 4096, False, False), (300, 200, 5000, True, False), (2048, 2048, 2048, True, False),
     (130, 70, 20000, False, True)],
)
def test_gemm_stream_k_splits(dev, M, N, K, ta, tb):
    # shapes whose tiles underfill the GPU: the k-iterations are split over
    # many workgroups and summed by the fixup kernel (several-way splits)
    from trnblas_amd.hip import kernels

    g = torch.Generator().manual_seed(M + K)
    A0 = torch.randn((K, M) if ta else (M, K), generator=g)
    B0 = torch.randn((N, K) if tb else (K, N), generator=g)
    C = torch.randn(M, N, generator=g)
    A = (A0.mT if ta else A0).to(dev)
    B = (B0.mT if tb else B0).to(dev)
    D1 = kernels.gemm(A, B, 1.0, 0.5, C.to(dev))
    D2 = kernels.gemm(A, B, 1.0, 0.5, C.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(D1, D2)  # deterministic
    err = _cw_err(D1.cpu(), A.cpu(), B.cpu(), 1.0, 0.5, C)
    assert err <= 1e-6, err


@pytest.mark.parametrize("n,k,uplo", [(4096, 1024, "lower"), (640, 9000, "upper")])
def test_syrk_stream_k(dev, n, k, uplo):
    from trnblas_amd.hip import kernels

    g = torch.Generator().manual_seed(n)
    A = torch.randn(n, k, generator=g)
    X = torch.randn(n, n, generator=g)
    D = kernels.syrk(A.to(dev), 1.0, 0.5, X.to(dev), uplo=uplo).cpu()
    assert torch.equal(D, D.T)
    Cs = torch.tril(X) + torch.tril(X, -1).T if uplo == "lower" else torch.triu(X) + torch.triu(X, 1).T
    Ad = A.double()
    ref = Ad @ Ad.T + 0.5 * Cs.double()
    den = Ad.abs() @ Ad.abs().T + 0.5 * Cs.double().abs()
    assert ((D.double() - ref).abs() / den).max().item() <= 1e-6


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 2.0**-8), (torch.float16, 2.0**-11)])
@pytest.mark.parametrize("n,k", [(384, 200), (300, 77)])
@pytest.mark.parametrize("uplo", ["lower", "upper"])
def test_syrk_16bit(dev, dtype, tol, n, k, uplo):
    # 16-bit SYRK: (384, 200) runs the direct-to-LDS kernel with whole
    # interior tiles (vector mirrored stores of 8 bytes), (300, 77) the
    # register-staged kernel with ragged edges. The only rounding beyond
    # fp32 accumulation is the final one to the 16-bit output.
    from trnblas_amd.hip import kernels

    g = torch.Generator().manual_seed(n * 7 + k)
    A = torch.randn(n, k, generator=g).to(dtype)
    X = torch.randn(n, n, generator=g).to(dtype)
    D = kernels.syrk(A.to(dev), 1.0, 0.5, X.to(dev), uplo=uplo).cpu()
    assert D.dtype == dtype and torch.equal(D, D.T)
    Xd = X.double()
    Cs = torch.tril(Xd) + torch.tril(Xd, -1).T if uplo == "lower" else torch.triu(Xd) + torch.triu(Xd, 1).T
    Ad = A.double()
    ref = Ad @ Ad.T + 0.5 * Cs
    den = Ad.abs() @ Ad.abs().T + 0.5 * Cs.abs()
    assert ((D.double() - ref).abs() / den).max().item() <= tol


def _tri_flags_ref(X):
    up = bool((torch.triu(X, 1) != 0).any())
    lo = bool((torch.tril(X, -1) != 0).any())
    return up, lo


@pytest.mark.parametrize("n", [1, 2, 77, 1024, 1500, 2100])
def test_triangle_nonzero_patterns(dev, n):
    # one pass of the device check against torch on patterns that make it
    # scan everything (empty triangles, a single entry in the far corner of
    # a triangle) and ones it decides early (filled C); NaN counts as nonzero
    from trnblas_amd.hip import kernels

    g = torch.Generator().manual_seed(n)
    full = torch.randn(n, n, generator=g)
    pats = {"full": full, "lower": torch.tril(full), "upper": torch.triu(full),
            "diag": torch.diag(torch.diagonal(full)), "zero": torch.zeros(n, n)}
    if n > 1:
        one_lo = torch.zeros(n, n)
        one_lo[n - 1, 0] = 3.0
        one_up = torch.zeros(n, n)
        one_up[0, n - 1] = float("nan")
        pats["corner_lo"] = one_lo
        pats["corner_up_nan"] = one_up
    for name, X in pats.items():
        for dtype in (torch.float32, torch.bfloat16):
            Xd = X.to(dtype).to(dev)
            for uplo in ("upper", "lower"):
                up, lo = _tri_flags_ref(X)
                want = (up, lo) if uplo == "upper" else (lo, up)
                assert kernels.triangle_nonzero(Xd, uplo) == want, (name, dtype, uplo)


@pytest.mark.parametrize("n,k", [(512, 96), (300, 77)])
@pytest.mark.parametrize("stored", ["full", "lower", "upper", "diag"])
@pytest.mark.parametrize("uplo", ["upper", "lower"])
def test_syrk_checked_triangle_rule(dev, n, k, stored, uplo):
    # the referenced triangle decided on the device: the flags returned and
    # the product must follow the host rule (level3.py:305-329)
    from trnblas_amd.hip import kernels

    g = torch.Generator().manual_seed(n + k)
    A = torch.randn(n, k, generator=g)
    full = torch.randn(n, n, generator=g)
    X = {"full": full, "lower": torch.tril(full), "upper": torch.triu(full),
         "diag": torch.diag(torch.diagonal(full))}[stored]
    D, mine, theirs = kernels.syrk_checked(A.to(dev), 1.0, 0.5, X.to(dev), uplo=uplo)
    up, lo = _tri_flags_ref(X)
    assert (mine, theirs) == ((up, lo) if uplo == "upper" else (lo, up))
    other = "lower" if uplo == "upper" else "upper"
    side = other if (theirs and not mine) else uplo
    D = D.cpu()
    assert torch.equal(D, D.T)
    Xd = X.double()
    Cs = torch.tril(Xd) + torch.tril(Xd, -1).T if side == "lower" else torch.triu(Xd) + torch.triu(Xd, 1).T
    Ad = A.double()
    ref = Ad @ Ad.T + 0.5 * Cs
    den = Ad.abs() @ Ad.abs().T + 0.5 * Cs.abs()
    assert ((D.double() - ref).abs() / den).max().item() <= 1e-6
    # the same product through the fixed-triangle entry point, bit for bit
    D2 = kernels.syrk(A.to(dev), 1.0, 0.5, X.to(dev), uplo=side).cpu()
    assert torch.equal(D, D2)


def test_syrk_unaligned_c_ld(dev):
    # a C whose leading dimension is not a multiple of 4 (no vector access
    # to C or D's mirror): the scalar epilogue, same values
    from trnblas_amd.hip import kernels

    n, k = 384, 64
    g = torch.Generator().manual_seed(5)
    A = torch.randn(n, k, generator=g).to(dev)
    big = torch.randn(n, n + 3, generator=g).to(dev)
    Xv = big[:, :n]  # ldc = n + 3
    D1 = kernels.syrk(A, 1.0, 0.5, Xv, uplo="upper")
    D2 = kernels.syrk(A, 1.0, 0.5, Xv.contiguous(), uplo="upper")
    torch.cuda.synchronize()
    assert torch.equal(D1, D2)


@pytest.mark.parametrize("M,N,K", [(128, 128, 32768), (256, 128, 20000), (1024, 1024, 1024), (64, 300, 4096)])
def test_gemm_stream_k_few_tiles(dev, M, N, K):
    # a handful of tiles with long K: every tile is split over many
    # workgroups (up to the fixup's 64 contributors per tile)
    from trnblas_amd.hip import kernels

    g = torch.Generator().manual_seed(M + N + K)
    A = torch.randn(M, K, generator=g)
    B = torch.randn(K, N, generator=g)
    C = torch.randn(M, N, generator=g)
    D1 = kernels.gemm(A.to(dev), B.to(dev), 1.0, 0.5, C.to(dev))
    D2 = kernels.gemm(A.to(dev), B.to(dev), 1.0, 0.5, C.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(D1, D2)  # deterministic
    err = _cw_err(D1.cpu(), A, B, 1.0, 0.5, C)
    assert err <= 1e-6, err


@pytest.mark.parametrize("n,k", [(128, 32768), (300, 8192)])
def test_syrk_stream_k_few_tiles(dev, n, k):
    from trnblas_amd.hip import kernels

    g = torch.Generator().manual_seed(n + k)
    A = torch.randn(n, k, generator=g)
    X = torch.randn(n, n, generator=g)
    D = kernels.syrk(A.to(dev), 1.0, 0.5, X.to(dev), uplo="upper").cpu()
    assert torch.equal(D, D.T)
    Cs = torch.triu(X) + torch.triu(X, 1).T
    Ad = A.double()
    ref = Ad @ Ad.T + 0.5 * Cs.double()
    den = Ad.abs() @ Ad.abs().T + 0.5 * Cs.double().abs()
    assert ((D.double() - ref).abs() / den).max().item() <= 1e-6



@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 2.0**-8), (torch.float16, 2.0**-11)])
@pytest.mark.parametrize(
    "batch,M,N,K",
    [(1, 4000, 2176, 1000), (16, 1000, 1024, 512), (1, 4096, 2176, 8192)],
)
def test_gemm_16bit_large(dev, dtype, tol, batch, M, N, K):
    # 16-bit A B^T (both K-contiguous) on aligned operands at sizes that fill
    # the GPU: ragged M, a batch, and (last) a stream-K tail; fp32
    # accumulation, one rounding to the 16-bit output
    from trnblas_amd.hip import kernels

    g = torch.Generator().manual_seed(M + K)
    A = torch.randn(batch, M, K, generator=g).to(dtype)
    Bt = torch.randn(batch, N, K, generator=g).to(dtype)
    C = torch.randn(batch, M, N, generator=g).to(dtype)
    Ad, Bd, Cd = A.to(dev), Bt.to(dev), C.to(dev)
    if batch == 1:
        Ad, Bd, Cd = Ad[0], Bd[0], Cd[0]
    D = kernels.gemm(Ad, Bd.mT, 1.0, 0.5, Cd)
    torch.cuda.synchronize()
    D = D.cpu().double().reshape(batch, M, N)
    ref = A.double() @ Bt.double().mT + 0.5 * C.double()
    den = A.double().abs() @ Bt.double().abs().mT + 0.5 * C.double().abs()
    assert ((D - ref).abs() / den).max().item() <= tol


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 2.0**-8), (torch.float16, 2.0**-11)])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_gemm_16bit_wide_tiles(dev, dtype, tol, ta, tb):
    # 16-bit GEMM on aligned operands whose 256 x 256 tiles fill every CU
    # (4000 x 4104: 16 x 17 tiles) with K of 8 k-tiles or more runs
    # hgemm256_kernel: every layout (K- or M/N-contiguous panels), ragged M,
    # N and K (520 = 8 k-tiles + 8), alpha and beta; a second call gives the
    # same bits
    from trnblas_amd.hip import kernels

    M, N, K = 4000, 4104, 520
    g = torch.Generator(device=dev).manual_seed(M + 7 * ta + 3 * tb)
    A = torch.randn(K, M, device=dev, generator=g).to(dtype).T if ta else torch.randn(M, K, device=dev, generator=g).to(dtype)
    B = torch.randn(N, K, device=dev, generator=g).to(dtype).T if tb else torch.randn(K, N, device=dev, generator=g).to(dtype)
    C = torch.randn(M, N, device=dev, generator=g).to(dtype)
    D = kernels.gemm(A, B, 0.75, 0.5, C)
    D2 = kernels.gemm(A, B, 0.75, 0.5, C)
    torch.cuda.synchronize()
    assert torch.equal(D, D2)
    Af, Bf, Cf = A.float(), B.float(), C.float()
    ref = 0.75 * (Af @ Bf) + 0.5 * Cf
    den = 0.75 * (Af.abs() @ Bf.abs()) + 0.5 * Cf.abs()
    assert ((D.float() - ref).abs() / den).max().item() <= tol


def test_stream_k_two_streams(dev):
    # split-k GEMMs launched on two streams may run at the same time: each
    # stream has its own partial-tile workspace, so both match the results
    # of the same calls made one after the other, bit for bit
    from trnblas_amd.hip import kernels

    g = torch.Generator(device=dev).manual_seed(11)
    ops = [(torch.randn(1024, 4096, device=dev, generator=g), torch.randn(4096, 1024, device=dev, generator=g))
           for _ in range(2)]
    want = [kernels.gemm(a, b) for a, b in ops]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(dev), torch.cuda.Stream(dev)]
    got = [[], []]
    for _ in range(4):
        for s, (a, b), out in zip(streams, ops, got):
            with torch.cuda.stream(s):
                out.append(kernels.gemm(a, b))
    torch.cuda.synchronize()
    for w, outs in zip(want, got):
        for o in outs:
            assert torch.equal(o, w)


def test_batched_stream_k_few_tiles(dev):
    # a batch of single-tile products with long K (split over many
    # workgroups per tile, partial tiles summed per batch entry), with a
    # stride-0 broadcast B and beta * C
    from trnblas_amd.hip import kernels

    g = torch.Generator().manual_seed(21)
    A = torch.randn(3, 100, 8192, generator=g)
    B = torch.randn(8192, 120, generator=g)
    C = torch.randn(3, 100, 120, generator=g)
    D = kernels.gemm(A.to(dev), B.to(dev).unsqueeze(0).expand(3, 8192, 120), 1.0, 0.5, C.to(dev))
    torch.cuda.synchronize()
    for b in range(3):
        err = _cw_err(D[b].cpu(), A[b], B, 1.0, 0.5, C[b])
        assert err <= 1e-6, (b, err)


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 2.0**-8), (torch.float16, 2.0**-11)])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_gemm_16bit_aligned_layouts(dev, dtype, tol, ta, tb):
    # 16-byte aligned rows in every layout: the direct-to-LDS kernel, whose
    # M/N-contiguous fragments use the transposing LDS read; ragged M and N
    from trnblas_amd.hip import kernels

    M, N, K = 392, 264, 512
    g = torch.Generator().manual_seed(7)
    A0 = torch.randn((K, M) if ta else (M, K), generator=g).to(dtype)
    B0 = torch.randn((N, K) if tb else (K, N), generator=g).to(dtype)
    C = torch.randn(M, N, generator=g).to(dtype)
    A = (A0.mT if ta else A0).to(dev)
    B = (B0.mT if tb else B0).to(dev)
    D = kernels.gemm(A, B, 1.5, -0.5, C.to(dev))
    torch.cuda.synchronize()
    Ad, Bd = A.cpu().double(), B.cpu().double()
    ref = 1.5 * (Ad @ Bd) - 0.5 * C.double()
    den = 1.5 * (Ad.abs() @ Bd.abs()) + 0.5 * C.double().abs()
    assert ((D.cpu().double() - ref).abs() / den).max().item() <= tol


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 2.0**-8), (torch.float16, 2.0**-11)])
def test_syrk_16bit_trans_aligned(dev, dtype, tol):
    # op(A) = A^T with A (k, n) N-contiguous and aligned: both SYRK panels
    # are M/N-contiguous (transposing LDS reads)
    from trnblas_amd.hip import kernels

    n, k = 392, 200
    g = torch.Generator().manual_seed(9)
    A = torch.randn(k, n, generator=g).to(dtype)
    X = torch.randn(n, n, generator=g).to(dtype)
    D = kernels.syrk(A.to(dev), 1.0, 0.5, X.to(dev), trans=True, uplo="lower").cpu()
    assert torch.equal(D, D.T)
    Ad, Xd = A.double().T, X.double()
    Cs = torch.tril(Xd) + torch.tril(Xd, -1).T
    ref = Ad @ Ad.T + 0.5 * Cs
    den = Ad.abs() @ Ad.abs().T + 0.5 * Cs.abs()
    assert ((D.double() - ref).abs() / den).max().item() <= tol


@pytest.mark.parametrize(
    "batch,M,N,K",
    [(1, 2048, 2048, 512), (1, 1900, 2100, 1000), (1, 2000, 1930, 700), (2, 1024, 2048, 768),
     (1, 2048, 2048, 2048), (1, 1024, 1024, 1024), (1, 512, 512, 8192), (1, 1280, 1272, 1280),
     (3, 256, 520, 2048), (1, 96, 200, 30000)],
)
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_gemm_narrow_tiles(dev, batch, M, N, K, ta, tb):
    # launches whose 128 x 128 tiles fill at most one slot per CU of the
    # MI355X's 256 CUs run the 128 x 64 kernel: whole tiles where they fill
    # one round of two slots per CU, else split by stream-K over 128 x 64
    # tiles (up to the fixup's 64 contributors at K = 30000): every layout,
    # ragged edges, a batch, alpha / beta, at the 1e-6 gate
    from trnblas_amd.hip import kernels

    g = torch.Generator().manual_seed(M + N + K + 2 * ta + tb)
    A = torch.randn(batch, K, M, generator=g).transpose(1, 2) if ta else torch.randn(batch, M, K, generator=g)
    B = torch.randn(batch, N, K, generator=g).transpose(1, 2) if tb else torch.randn(batch, K, N, generator=g)
    C = torch.randn(batch, M, N, generator=g)
    if batch == 1:
        D = kernels.gemm(A[0].to(dev), B[0].to(dev), 1.5, -0.5, C[0].to(dev)).unsqueeze(0)
    else:
        D = kernels.gemm(A.to(dev), B.to(dev), 1.5, -0.5, C.to(dev))
    torch.cuda.synchronize()
    err = max(_cw_err(D[b].cpu(), A[b], B[b], 1.5, -0.5, C[b]) for b in range(batch))
    assert err <= 1e-6, err


@pytest.mark.parametrize("batch,M,N,K", [(1, 2048, 2048, 2048), (2, 1024, 2048, 1024), (1, 1900, 2100, 1037), (1, 2040, 2044, 3000)])
def test_gemm_pipe_kernel_transposed_a(dev, batch, M, N, K):
    # A^T B with one round of 128 x 128 tiles over the CUs and K >= 1024 runs
    # the one-workgroup-per-CU kernel (compute waves + operand movers): a
    # batch, ragged M / N / K, C broadcast over the batch with an odd row
    # stride (scalar epilogue), alpha / beta, deterministic, at the 1e-6 gate
    from trnblas_amd.hip import kernels

    g = torch.Generator().manual_seed(M + N + K + batch)
    A = torch.randn(batch, K, M, generator=g).transpose(1, 2)
    B = torch.randn(batch, K, N, generator=g)
    Cw = torch.randn(M, N + 1, generator=g)
    C = Cw[:, :N]
    Ad, Bd, Cd = A.to(dev), B.to(dev), Cw.to(dev)[:, :N]
    if batch == 1:
        D = kernels.gemm(Ad[0], Bd[0], 0.75, 0.5, Cd).unsqueeze(0)
        D2 = kernels.gemm(Ad[0], Bd[0], 0.75, 0.5, Cd).unsqueeze(0)
    else:
        D = kernels.gemm(Ad, Bd, 0.75, 0.5, Cd)
        D2 = kernels.gemm(Ad, Bd, 0.75, 0.5, Cd)
    torch.cuda.synchronize()
    assert torch.equal(D, D2)
    err = max(_cw_err(D[b].cpu(), A[b], B[b], 0.75, 0.5, C) for b in range(batch))
    assert err <= 1e-6, err


@pytest.mark.parametrize("dtype,tol", [(torch.bfloat16, 2.0**-8), (torch.float16, 2.0**-10)])
@pytest.mark.parametrize("M,N,K", [(1024, 1024, 4096), (1280, 1272, 1280), (512, 520, 8192), (2048, 2048, 2048)])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_gemm_16bit_narrow_tiles(dev, dtype, tol, M, N, K, ta, tb):
    # 16-bit launches with at most one 128 x 128 tile per CU and >= 20
    # 64-wide k-tiles run the 128 x 64 kernel (stream-K where the grid is
    # small); every layout, a ragged edge, against fp64 of the rounded inputs
    from trnblas_amd.hip import kernels

    g = torch.Generator().manual_seed(M + N + K + 2 * ta + tb)
    A = (torch.randn(K, M, generator=g).T if ta else torch.randn(M, K, generator=g)).to(dtype)
    B = (torch.randn(N, K, generator=g).T if tb else torch.randn(K, N, generator=g)).to(dtype)
    C = torch.randn(M, N, generator=g).to(dtype)
    D = kernels.gemm(A.to(dev), B.to(dev), 1.0, 0.5, C.to(dev)).cpu()
    ref = A.double() @ B.double() + 0.5 * C.double()
    den = A.double().abs() @ B.double().abs() + 0.5 * C.double().abs()
    assert ((D.double() - ref).abs() / den).max().item() <= tol


def _misaligned(X, dev):
    # X on the device one element past a 16-byte boundary (same values)
    buf = torch.empty(X.numel() + 1, dtype=X.dtype, device=dev)
    Y = buf[1:].view(X.shape)
    Y.copy_(X.to(dev))
    return Y


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-6), (torch.bfloat16, 2.0**-8)])
@pytest.mark.parametrize(
    "batch,bb,M,N,K,shift",
    [(1, 1, 37, 53, 71, False), (1, 1, 130, 257, 1001, False), (1, 1, 1, 5, 3, False),
     (1, 1, 200, 64, 3, False), (1, 1, 128, 128, 128, True), (1, 1, 129, 130, 517, True),
     (3, 1, 65, 70, 33, False), (4, 4, 96, 33, 250, False)],
)
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_gemm_packed_operands(dev, monkeypatch, dtype, tol, batch, bb, M, N, K, shift, ta, tb):
    # operands the DMA kernel cannot read in place (ragged contiguous
    # extents, K not a multiple of 16 bytes, a base one element off a
    # 16-byte boundary) packed into zero-padded K-contiguous buffers at
    # every size (threshold 0): every layout, a batch (B broadcast or not),
    # alpha / beta, against fp64 at the north-star gate
    from trnblas_amd.hip import kernels

    monkeypatch.setattr(kernels, "PACK_MIN_MACS", {4: 0, 2: 0})
    packs = []
    orig = kernels._pack_k
    monkeypatch.setattr(kernels, "_pack_k", lambda X, kp: packs.append(kp) or orig(X, kp))
    g = torch.Generator().manual_seed(M + 3 * N + 7 * K + batch + 2 * ta + tb)
    A = torch.randn(batch, K, M, generator=g).transpose(1, 2) if ta else torch.randn(batch, M, K, generator=g)
    B = torch.randn(bb, N, K, generator=g).transpose(1, 2) if tb else torch.randn(bb, K, N, generator=g)
    A, B = A.to(dtype), B.to(dtype)
    C = torch.randn(batch, M, N, generator=g).to(dtype)
    if batch == 1:
        Ad, Bd = A[0].to(dev), B[0].to(dev)
        if shift:
            Ad = _misaligned(A[0].mT.contiguous(), dev).mT if ta else _misaligned(A[0], dev)
        D = kernels.gemm(Ad, Bd, 1.5, -0.5, C[0].to(dev)).unsqueeze(0).cpu()
    else:
        D = kernels.gemm(A.to(dev), B.to(dev), 1.5, -0.5, C.to(dev)).cpu()
    ev = 16 // A.element_size()
    # an operand is packed exactly when it is not DMA-ready in place
    assert bool(packs) == bool(shift or (M if ta else K) % ev or (K if tb else N) % ev)
    for b in range(batch):
        Ab, Bb = A[b].double(), B[min(b, bb - 1)].double()
        ref = 1.5 * (Ab @ Bb) - 0.5 * C[b].double()
        den = 1.5 * (Ab.abs() @ Bb.abs()) + 0.5 * C[b].double().abs()
        den = torch.where(den > 0, den, torch.ones_like(den))
        assert ((D[b].double() - ref).abs() / den).max().item() <= tol


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-6), (torch.bfloat16, 2.0**-8)])
@pytest.mark.parametrize("M,N,K,ta,tb", [(1537, 1539, 1541, False, False), (2047, 1025, 1027, True, True),
                                         (1023, 2049, 1031, False, True)])
def test_gemm_unaligned_large(dev, dtype, tol, M, N, K, ta, tb):
    # products above the packing threshold with odd extents take the DMA
    # kernel on packed operands (at the default threshold)
    from trnblas_amd.hip import kernels

    assert M * N * K >= kernels.PACK_MIN_MACS[4]
    g = torch.Generator().manual_seed(M + N + K)
    A = (torch.randn(K, M, generator=g).T if ta else torch.randn(M, K, generator=g)).to(dtype)
    B = (torch.randn(N, K, generator=g).T if tb else torch.randn(K, N, generator=g)).to(dtype)
    C = torch.randn(M, N, generator=g).to(dtype)
    D = kernels.gemm(A.to(dev), B.to(dev), 1.0, 0.5, C.to(dev)).cpu()
    ref = A.double() @ B.double() + 0.5 * C.double()
    den = A.double().abs() @ B.double().abs() + 0.5 * C.double().abs()
    assert ((D.double() - ref).abs() / den).max().item() <= tol


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-6), (torch.bfloat16, 2.0**-8)])
@pytest.mark.parametrize("n,k", [(130, 1001), (257, 33), (1, 3), (2047, 1027)])
@pytest.mark.parametrize("trans", [False, True])
def test_syrk_packed_operand(dev, monkeypatch, dtype, tol, n, k, trans):
    # SYRK on an operand packed K-contiguous with k padded (threshold 0)
    from trnblas_amd.hip import kernels

    monkeypatch.setattr(kernels, "PACK_MIN_MACS", {4: 0, 2: 0})
    g = torch.Generator().manual_seed(n + k + trans)
    A = torch.randn((k, n) if trans else (n, k), generator=g).to(dtype)
    X = torch.randn(n, n, generator=g).to(dtype)
    D = kernels.syrk(A.to(dev), 1.0, 0.5, X.to(dev), trans=trans, uplo="lower").cpu()
    assert torch.equal(D, D.T)
    opA = (A.T if trans else A).double()
    Xd = X.double()
    Cs = torch.tril(Xd) + torch.tril(Xd, -1).T
    ref = opA @ opA.T + 0.5 * Cs
    den = opA.abs() @ opA.abs().T + 0.5 * Cs.abs()
    assert ((D.double() - ref).abs() / den).max().item() <= tol


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("R,K,kp", [(1, 1, 4), (64, 64, 64), (65, 63, 72), (130, 257, 264), (3, 1000, 1008)])
@pytest.mark.parametrize("layout", ["row", "trans", "strided", "batched", "broadcast"])
def test_pack_k_kernel(dev, dtype, R, K, kp, layout):
    # trnblas_hip_pack_k copies bits exactly and zero-fills columns K .. kp - 1
    # for a row-major source, a transposed view, a general strided view
    # (every other row and column), a batch, and a stride-0 batch
    from trnblas_amd.hip import kernels

    g = torch.Generator().manual_seed(R * 3 + K + kp)
    if layout == "row":
        X = torch.randn(R, K, generator=g).to(dtype).to(dev)
    elif layout == "trans":
        X = torch.randn(K, R, generator=g).to(dtype).to(dev).T
    elif layout == "strided":
        X = torch.randn(2 * R, 2 * K, generator=g).to(dtype).to(dev)[::2, ::2]
    elif layout == "batched":
        X = torch.randn(3, K, R, generator=g).to(dtype).to(dev).transpose(1, 2)
    else:
        X = torch.randn(1, R, K, generator=g).to(dtype).to(dev).expand(2, R, K)
    P = kernels._pack_k(X, kp)
    ref = torch.zeros((*X.shape[:-1], kp), dtype=dtype, device=dev)
    ref[..., :K] = X
    torch.cuda.synchronize()
    assert P.shape == ref.shape and P.is_contiguous()
    assert torch.equal(P.view(torch.int16 if dtype != torch.float32 else torch.int32),
                       ref.view(torch.int16 if dtype != torch.float32 else torch.int32))
