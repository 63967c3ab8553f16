"""trnblas_hip_pair_energy_noalloc (the entry point that allocates nothing:
its partials live in a static device array) against trnblas_hip_pair_energy
(caller workspace), both called through the C ABI: the same kernels, so the
same bits. Two calls in a row, the second smaller, in both pair modes, and
the size limit reported as an error."""

import ctypes

import pytest
import torch

from trnblas_amd import df_mp2
from trnblas_amd.hip import _lib

pytestmark = pytest.mark.gpu


def _inputs(dev, nocc, nvir, naux, seed):
    B, eo, ev = df_mp2.pair_inputs(nocc, nvir, naux, seed=seed)
    return B.to(dev).contiguous(), eo.to(dev).float(), ev.to(dev).float()


def _both(dev, B, eo, ev, pairs=None):
    """(out_pairs, out_total) from the workspace entry point and from the
    no-allocation one, on the same inputs."""
    lib = _lib.load()
    nocc, nvir, naux = B.shape
    if pairs is None:
        npairs, pi, pj = nocc * (nocc + 1) // 2, None, None
    else:
        pi = torch.tensor([p[0] for p in pairs], dtype=torch.int32, device=dev)
        pj = torch.tensor([p[1] for p in pairs], dtype=torch.int32, device=dev)
        npairs = len(pairs)
    s = _lib.stream_of(dev)
    ld_occ, ld_vir = B.stride(0), B.stride(1)
    head = (nvir, naux, B.data_ptr(), ld_occ, B.data_ptr(), ld_occ, ld_vir,
            eo.data_ptr(), eo.data_ptr(), ev.data_ptr(), nocc, npairs, _lib.ptr(pi), _lib.ptr(pj), None)
    outs = []
    for entry in ("trnblas_hip_pair_energy", "trnblas_hip_pair_energy_noalloc"):
        e_pairs = torch.full((npairs,), float("nan"), dtype=torch.float64, device=dev)
        total = torch.full((), float("nan"), dtype=torch.float64, device=dev)
        if entry == "trnblas_hip_pair_energy":
            ws = lib.trnblas_hip_pair_energy_workspace(nvir, npairs)
            work = torch.empty(max(ws, 8), dtype=torch.uint8, device=dev)
            _lib.call(entry, *head, e_pairs.data_ptr(), total.data_ptr(), work.data_ptr(), work.numel(), s)
        else:
            _lib.call(entry, *head, e_pairs.data_ptr(), total.data_ptr(), s)
        torch.cuda.synchronize()
        outs.append((e_pairs.cpu(), float(total)))
    return outs


def test_noalloc_matches_workspace_entry_two_calls(dev):
    # first call: C3-like shape (every pair i <= j); second: smaller, so stale
    # partials of the first call sit beyond what the second one reads
    for nocc, nvir, naux, seed in ((24, 200, 256, 1), (5, 97, 130, 2)):
        B, eo, ev = _inputs(dev, nocc, nvir, naux, seed)
        (p_ws, t_ws), (p_na, t_na) = _both(dev, B, eo, ev)
        assert torch.equal(p_na, p_ws), (nocc, nvir)
        assert t_na == t_ws, (nocc, nvir, t_na, t_ws)
        assert t_na != 0.0 and t_na == t_na


def test_noalloc_explicit_pairs_and_empty(dev):
    B, eo, ev = _inputs(dev, 9, 150, 200, 3)
    pairs = [(0, 0), (3, 7), (8, 1), (5, 5), (2, 8)]
    (p_ws, t_ws), (p_na, t_na) = _both(dev, B, eo, ev, pairs)
    assert torch.equal(p_na, p_ws)
    assert t_na == t_ws
    # nocc == 0: zero energy, written by the entry point (no memset)
    E, eo0, ev0 = _inputs(dev, 1, 150, 200, 4)
    (_, t0_ws), (_, t0_na) = _both(dev, E[:0], eo0[:0], ev0)
    assert t0_na == 0.0 and t0_ws == 0.0


def test_noalloc_rejects_calls_beyond_its_scratch(dev):
    lib = _lib.load()
    cap = lib.trnblas_hip_pair_energy_noalloc_max_bytes()
    assert cap == 16 << 20
    # nocc 512 at nvir 768: 131328 pairs x 37 partials x 8 B = 38.9 MB > 16 MiB.
    # The size check comes before any launch, so the operands may be tiny.
    x = torch.zeros(8, device=dev)
    rc = lib.trnblas_hip_pair_energy_noalloc(768, 1, x.data_ptr(), 768, x.data_ptr(), 768, 1,
                                             x.data_ptr(), x.data_ptr(), x.data_ptr(), 512, 0,
                                             None, None, None, None, x.data_ptr(),
                                             ctypes.c_void_p(_lib.stream_of(dev)))
    assert rc == _lib.E_WORKSPACE
    assert b"static scratch" in lib.trnblas_hip_last_error()
