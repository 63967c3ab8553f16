"""The fp16x3 operand split, bit for bit: after a trnblas_hip_pair_energy_fp16x3
call (the implicit i <= j walk, caller workspace) the workspace holds the
pieces of B and the row exponents, in the layout the C ABI documents
(include/trnblas_hip.h, trnblas_hip_pair_energy_fp16x3_workspace). They are
checked against a numpy statement of the split:

  e(o, a) = 15 - E for the row's largest magnitude f 2^E, f in [0.5, 1)
            (0 for a zero row and for the padding row of an odd nvir),
  xs = x 2^e,  hi = rn_f16(xs),  lo = rn_f16(xs - hi),

element (o, a, p, k) at ((((o nvp + a / 2) nk + k / 32) 2 + p) 2 + a % 2) 32
+ k % 32 with nvp = ceil(nvir / 2), nk = ldv / 32, ldv = naux rounded up to
64, zeros in the padding. The numpy statement is itself pinned by the split's
invariants (largest scaled magnitude in [2^14, 2^15), hi + lo within 2^-11 of
an fp16 ulp of hi, lo no larger than half an ulp of hi). The split has no
counterpart in the reference (its energy runs in fp32 on the NKI engines);
it is this library's arithmetic, so the format itself is the oracle here.
The bf16x6 split (three round-to-nearest bf16 pieces, hi + mid + lo == x
exactly) is checked the same way through trnblas_hip_pair_energy_bf16x6.
"""

import numpy as np
import pytest
import torch

from trnblas_amd.hip import _lib

pytestmark = pytest.mark.gpu


def _al256(n):
    return (n + 255) // 256 * 256


def _expected(B):
    nocc, nvir, naux = B.shape
    ldv = -(-naux // 64) * 64
    nvp, nk = (nvir + 1) // 2, ldv // 32
    X = np.zeros((nocc, 2 * nvp, ldv), np.float32)
    X[:, :nvir, :naux] = B
    m = np.abs(X).max(axis=2)
    _, ex = np.frexp(m)
    e = np.where(m > 0, 15 - ex, 0).astype(np.int32)
    xs = np.ldexp(X, e[:, :, None]).astype(np.float32)
    hi = xs.astype(np.float16)
    lo = (xs - hi.astype(np.float32)).astype(np.float16)
    # the split's invariants
    nz = m > 0
    top = np.abs(xs).max(axis=2)
    assert np.all((top[nz] >= 2.0**14) & (top[nz] < 2.0**15))
    ulp = np.spacing(np.abs(hi)).astype(np.float32)  # fp16 spacing at hi
    assert np.all(np.abs(lo.astype(np.float32)) <= ulp / 2)
    res = np.abs(xs - hi.astype(np.float32) - lo.astype(np.float32))
    assert np.all(res <= np.maximum(ulp * 2.0**-11, np.float32(2.0**-25)))
    # (o, a, p, k) -> ((((o nvp + a / 2) nk + k / 32) 2 + p) 2 + a % 2) 32 + k % 32
    pieces = np.stack([hi, lo], axis=2)  # (o, a, p, k)
    pieces = pieces.reshape(nocc, nvp, 2, 2, nk, 32)  # (o, m, d, p, s, c)
    P = pieces.transpose(0, 1, 4, 3, 2, 5).reshape(-1)  # (o, m, s, p, d, c)
    return P.view(np.uint16), e.reshape(-1), ldv


def _run(dev, B, math="fp16x3"):
    npc = 2 if math == "fp16x3" else 3
    lib = _lib.load()
    nocc, nvir, naux = B.shape
    npairs = nocc * (nocc + 1) // 2
    g = torch.Generator().manual_seed(1)
    eo = (-1.5 + 1.2 * torch.rand(nocc, generator=g)).to(dev)
    ev = (0.1 + 2.9 * torch.rand(nvir, generator=g)).to(dev)
    ws = getattr(lib, f"trnblas_hip_pair_energy_{math}_workspace")(nvir, naux, npairs, nocc, 0)
    work = torch.zeros(ws, dtype=torch.uint8, device=dev)
    total = torch.full((), float("nan"), dtype=torch.float64, device=dev)
    Bd = B.to(dev)
    _lib.call(f"trnblas_hip_pair_energy_{math}", nvir, naux, Bd.data_ptr(), nocc, Bd.stride(0),
              Bd.data_ptr(), 0, Bd.stride(0), Bd.stride(1), eo.data_ptr(), eo.data_ptr(), ev.data_ptr(),
              nocc, npairs, None, None, None, None, total.data_ptr(), work.data_ptr(), work.numel(),
              _lib.stream_of(dev))  # fmt: skip
    torch.cuda.synchronize()
    assert np.isfinite(float(total))
    w = work.cpu().numpy()
    base = _al256(lib.trnblas_hip_pair_energy_workspace(nvir, npairs))
    ldv = -(-naux // 64) * 64
    nvp = (nvir + 1) // 2
    pbytes = 2 * npc * nocc * nvp * ldv * 2
    P = w[base : base + pbytes].view(np.uint16)
    if npc == 3:
        return P, None
    eb = base + _al256(pbytes)
    E = w[eb : eb + nocc * 2 * nvp * 4].view(np.int32)
    return P, E


@pytest.mark.parametrize(
    "nocc, nvir, naux, kind",
    [
        (3, 7, 33, "plain"),  # odd nvir (a padding row), ragged naux, unaligned rows
        (4, 10, 128, "plain"),  # 16-byte rows: the vector load path
        (5, 9, 96, "wide"),  # rows 2^-30 .. 2^20 apart, one zero row
        (2, 1, 300, "plain"),  # one virtual row: every pair half padding
    ],
)
def test_fp16x3_split_bit_exact(dev, nocc, nvir, naux, kind):
    print(f"split case nocc {nocc} nvir {nvir} naux {naux} {kind}", flush=True)
    g = torch.Generator().manual_seed(nocc * 100 + nvir)
    B = 0.05 * torch.randn(nocc, nvir, naux, generator=g)
    if kind == "wide":
        B = B * torch.pow(2.0, torch.randint(-30, 21, (nocc, nvir, 1), generator=g).float())
        B[1, 4] = 0.0
    P, E = _run(dev, B)
    Pe, Ee, _ = _expected(B.numpy())
    np.testing.assert_array_equal(E, Ee)
    bad = np.flatnonzero(P != Pe)
    assert bad.size == 0, f"{bad.size} of {P.size} pieces differ, first at {bad[:8]}"


def _expected_bf16x6(B):
    """hi = rn_bf16(x), mid = rn_bf16(x - hi), lo = rn_bf16(x - hi - mid)
    (fp32 differences, exact), in the same row-pair layout with three pieces."""
    nocc, nvir, naux = B.shape
    ldv = -(-naux // 64) * 64
    nvp, nk = (nvir + 1) // 2, ldv // 32
    X = torch.zeros(nocc, 2 * nvp, ldv)
    X[:, :nvir, :naux] = B
    hi = X.to(torch.bfloat16)
    r = X - hi.float()
    mid = r.to(torch.bfloat16)
    r2 = r - mid.float()
    lo = r2.to(torch.bfloat16)
    # every normal x is exactly hi + mid + lo
    assert torch.equal(hi.double() + mid.double() + lo.double(), X.double())
    pieces = torch.stack([hi, mid, lo], dim=2).view(torch.int16).numpy()  # (o, a, p, k)
    pieces = pieces.reshape(nocc, nvp, 2, 3, nk, 32)  # (o, m, d, p, s, c)
    return pieces.transpose(0, 1, 4, 3, 2, 5).reshape(-1).view(np.uint16)


@pytest.mark.parametrize("nocc, nvir, naux", [(3, 7, 33), (4, 10, 128), (2, 1, 300)])
def test_bf16x6_split_bit_exact(dev, nocc, nvir, naux):
    print(f"bf16x6 split case nocc {nocc} nvir {nvir} naux {naux}", flush=True)
    g = torch.Generator().manual_seed(nocc * 100 + nvir + 7)
    B = 0.05 * torch.randn(nocc, nvir, naux, generator=g)
    P, _ = _run(dev, B, "bf16x6")
    Pe = _expected_bf16x6(B)
    bad = np.flatnonzero(P != Pe)
    assert bad.size == 0, f"{bad.size} of {P.size} pieces differ, first at {bad[:8]}"
