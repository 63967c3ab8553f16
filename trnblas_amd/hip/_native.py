"""The `torch.ops.trnblas.*` custom-op surface, on the gfx950 kernels.

Same 20 op names, argument shapes and result shapes/dtypes as the
reference's registration (trnblas/nki/_native.py:49-259, names at
:243-259), each registered with `torch.library.custom_op` (functional:
`mutates_args=()`, one fresh Tensor out) for the CUDA (= ROCm) device and
with a fake (meta) function giving the reference's output shape, so
`torch.compile` can trace calls. Every entry of `OPS` is wrapped by the
operand-dtype backstop (`dispatch._check_kernel_operands`, TypeError).

Importing this module registers the ops; `dispatch.get_native_ops()`
imports it on first use only (importing `trnblas_amd` registers nothing and
loads no library).

The reference's ops return per-partition partial sums that the host adds up
(`partial.sum()`); here the energy ops compute each pair's energy in fp64
on the device and return it in row 0 of the same-shaped fp32 result (the
other rows zero), so `partial.sum()` — and any caller that sums the columns
— gets the same totals.
"""

import torch
from torch import Tensor

from . import kernels
from .dispatch import _check_kernel_operands

_PAIR_TILE = 128  # partition rows of the reference's energy-op outputs


def _mp2_p_tile(nvir: int) -> int:
    p = min(nvir, 128)
    while p > 1 and nvir % p != 0:
        p -= 1
    return max(p, 1)


def _rows(values: Tensor, rows: int, dtype=torch.float32) -> Tensor:
    """(rows, n) result with `values` in row 0 and zeros below."""
    out = torch.zeros((rows, values.numel()), dtype=dtype, device=values.device)
    out[0] = values.to(dtype)
    return out


# ── GEMM family: every tile name is the same gfx950 kernel ───────────────────

_GEMM_NAMES = [
    f"gemm_{tm}_{tk}_{tn}"
    for tm, tk, tn in ((64, 128, 128), (64, 128, 256), (64, 128, 512),
                       (128, 128, 128), (128, 128, 256), (128, 128, 512))
] + ["gemm_ragged", "gemm_lnc"]  # fmt: skip


def _register_gemm(name: str):
    def impl(a: Tensor, b: Tensor) -> Tensor:
        return kernels.gemm(a, b)

    op = torch.library.custom_op(f"trnblas::{name}", impl, mutates_args=(), device_types="cuda")

    @op.register_fake
    def _(a, b):
        return a.new_empty((a.shape[0], b.shape[1]))

    return op


@torch.library.custom_op("trnblas::gemm_lnc_tn", mutates_args=(), device_types="cuda")
def gemm_lnc_tn(at: Tensor, b: Tensor) -> Tensor:
    return kernels.gemm(at.mT, b)  # the transposed operand is read in place


@gemm_lnc_tn.register_fake
def _(at, b):
    return at.new_empty((at.shape[1], b.shape[1]))


@torch.library.custom_op("trnblas::syrk", mutates_args=(), device_types="cuda")
def syrk(a: Tensor) -> Tensor:
    return kernels.syrk(a)


@syrk.register_fake
def _(a):
    return a.new_empty((a.shape[0], a.shape[0]))


# ── DF-MP2 energy ops ────────────────────────────────────────────────────────


@torch.library.custom_op("trnblas::mp2_energy", mutates_args=(), device_types="cuda")
def mp2_energy(
    t_flat: Tensor,
    eps_occ_chunk: Tensor,
    eps_occ_full: Tensor,
    eps_vir_col: Tensor,
    eps_vir_row: Tensor,
) -> Tensor:
    e = kernels.mp2_energy_pairs(
        t_flat, eps_occ_chunk.reshape(-1), eps_occ_full.reshape(-1), eps_vir_row.reshape(-1)
    )
    return _rows(e, _mp2_p_tile(eps_vir_row.shape[1]))


@mp2_energy.register_fake
def _(t_flat, eps_occ_chunk, eps_occ_full, eps_vir_col, eps_vir_row):
    return t_flat.new_empty(
        (_mp2_p_tile(eps_vir_row.shape[1]), eps_occ_chunk.shape[1] * eps_occ_full.shape[1]),
        dtype=torch.float32,
    )


@torch.library.custom_op("trnblas::fused_gemm_energy", mutates_args=(), device_types="cuda")
def fused_gemm_energy(
    b_i: Tensor, b_j: Tensor, eps_occ_sum: Tensor, eps_vir_col: Tensor, eps_vir_row: Tensor
) -> Tensor:
    zero = torch.zeros(1, dtype=torch.int32, device=b_i.device)
    eo = eps_occ_sum.reshape(1).to(torch.float32)
    e = kernels.pair_energies(
        b_i.unsqueeze(0), b_j.unsqueeze(0), eo, torch.zeros_like(eo),
        eps_vir_row.reshape(-1), zero, zero,
    )  # fmt: skip
    out = torch.zeros((b_i.shape[0], 1), dtype=torch.float32, device=b_i.device)
    out[0, 0] = e[0].to(torch.float32)
    return out


@fused_gemm_energy.register_fake
def _(b_i, b_j, eps_occ_sum, eps_vir_col, eps_vir_row):
    return b_i.new_empty((b_i.shape[0], 1), dtype=torch.float32)


def _upper_pairs(n: int, device) -> tuple[Tensor, Tensor]:
    iu = torch.triu_indices(n, n, device=device)
    return iu[0].to(torch.int32), iu[1].to(torch.int32)


@torch.library.custom_op("trnblas::batched_pair", mutates_args=(), device_types="cuda")
def batched_pair(B: Tensor, eps_occ_row: Tensor, eps_vir_col: Tensor, eps_vir_row: Tensor) -> Tensor:
    nocc = B.shape[0]
    eo = eps_occ_row.reshape(-1)
    pi, pj = _upper_pairs(nocc, B.device)
    e = kernels.pair_energies(B, B, eo, eo, eps_vir_row.reshape(-1), pi, pj)
    full = torch.zeros((nocc, nocc), dtype=torch.float64, device=B.device)
    full[pi.long(), pj.long()] = e
    full[pj.long(), pi.long()] = e  # e_ji = e_ij
    return _rows(full.reshape(-1), _PAIR_TILE)


@batched_pair.register_fake
def _(B, eps_occ_row, eps_vir_col, eps_vir_row):
    return B.new_empty((_PAIR_TILE, B.shape[0] * B.shape[0]), dtype=torch.float32)


@torch.library.custom_op("trnblas::j_batched", mutates_args=(), device_types="cuda")
def j_batched(
    b_i: Tensor,
    B: Tensor,
    eps_occ_i: Tensor,
    eps_occ_row: Tensor,
    eps_vir_col: Tensor,
    eps_vir_row: Tensor,
) -> Tensor:
    nocc = B.shape[0]
    pj = torch.arange(nocc, dtype=torch.int32, device=B.device)
    pi = torch.zeros_like(pj)
    e = kernels.pair_energies(
        b_i.unsqueeze(0), B, eps_occ_i.reshape(1), eps_occ_row.reshape(-1),
        eps_vir_row.reshape(-1), pi, pj,
    )  # fmt: skip
    return _rows(e, _PAIR_TILE)


@j_batched.register_fake
def _(b_i, B, eps_occ_i, eps_occ_row, eps_vir_col, eps_vir_row):
    return B.new_empty((_PAIR_TILE, B.shape[0]), dtype=torch.float32)


@torch.library.custom_op("trnblas::pair_energy_sym", mutates_args=(), device_types="cuda")
def pair_energy_sym(
    bt_i: Tensor,
    Bw: Tensor,
    eps_occ_i: Tensor,
    eps_occ_w: Tensor,
    eps_vir_col: Tensor,
    eps_vir_row: Tensor,
) -> Tensor:
    nd = Bw.shape[0]
    # bt_i = B[i]^T (naux, nvir), Bw[d] = B[j_d]^T: back to (nvir, naux) rows
    bi = bt_i.mT.unsqueeze(0)
    bj = Bw.transpose(1, 2)
    pj = torch.arange(nd, dtype=torch.int32, device=Bw.device)
    e = kernels.pair_energies(
        bi, bj, eps_occ_i.reshape(1), eps_occ_w.reshape(-1), eps_vir_row.reshape(-1),
        torch.zeros_like(pj), pj,
    )  # fmt: skip
    return _rows(e, _PAIR_TILE)


@pair_energy_sym.register_fake
def _(bt_i, Bw, eps_occ_i, eps_occ_w, eps_vir_col, eps_vir_row):
    return Bw.new_empty((_PAIR_TILE, Bw.shape[0]), dtype=torch.float32)


# ── Ozaki ops (reference layouts: bf16 digits, raw int32 bits) ───────────────


def _as_f64(xw: Tensor) -> Tensor:
    return xw.contiguous().view(torch.float64)


@torch.library.custom_op("trnblas::ozaki_gemm", mutates_args=(), device_types="cuda")
def ozaki_gemm(at: Tensor, b: Tensor) -> Tensor:
    k, Kp, Mp = at.shape
    N = b.shape[2]
    da = at.to(torch.int8).transpose(1, 2).contiguous()  # (k, Mp, Kp)
    db = b.to(torch.int8).transpose(1, 2).contiguous()  # (k, N, Kp)
    return kernels.ozaki_hilo(da, db, Mp, N, k)


@ozaki_gemm.register_fake
def _(at, b):
    return at.new_empty((2, at.shape[2], b.shape[2]), dtype=torch.float32)


def _exp_field(xw: Tensor) -> Tensor:
    return (xw[:, 1::2] >> 20) & 0x7FF  # biased fp64 exponent of each element


@torch.library.custom_op("trnblas::ozaki_emax", mutates_args=(), device_types="cuda")
def ozaki_emax(xw: Tensor) -> Tensor:
    f = _exp_field(xw)
    if f.shape[1] == 0:
        return torch.zeros((xw.shape[0], 1), dtype=torch.float32, device=xw.device)
    return f.amax(dim=1, keepdim=True).to(torch.float32)


@ozaki_emax.register_fake
def _(xw):
    return xw.new_empty((xw.shape[0], 1), dtype=torch.float32)


@torch.library.custom_op("trnblas::ozaki_emax_col", mutates_args=(), device_types="cuda")
def ozaki_emax_col(xw: Tensor) -> Tensor:
    f = _exp_field(xw)
    if f.shape[0] == 0:
        return torch.zeros((1, f.shape[1]), dtype=torch.float32, device=xw.device)
    return f.amax(dim=0, keepdim=True).to(torch.float32)


@ozaki_emax_col.register_fake
def _(xw):
    return xw.new_empty((1, xw.shape[1] // 2), dtype=torch.float32)


def _split_padded(xw: Tensor, k: int, per: str) -> Tensor:
    X = _as_f64(xw)
    R, C = X.shape
    rp, cp = -(-R // 128) * 128, -(-C // 128) * 128
    d, _, _ = kernels.ozaki_split(X, k, per)
    if per == "col":
        d = d.transpose(1, 2)  # (k, Kp=Rp, Cp) -> back to X's layout (k, Rp, Cp)
    return d[:, :rp, :cp].to(torch.bfloat16).contiguous()


@torch.library.custom_op("trnblas::ozaki_split", mutates_args=(), device_types="cuda")
def ozaki_split(xw: Tensor, rcs: Tensor) -> Tensor:
    return _split_padded(xw, rcs.shape[1], "row")


@ozaki_split.register_fake
def _(xw, rcs):
    rp = -(-xw.shape[0] // 128) * 128
    cp = -(-(xw.shape[1] // 2) // 128) * 128
    return xw.new_empty((rcs.shape[1], rp, cp), dtype=torch.bfloat16)


@torch.library.custom_op("trnblas::ozaki_split_col", mutates_args=(), device_types="cuda")
def ozaki_split_col(xw: Tensor, rcs: Tensor) -> Tensor:
    return _split_padded(xw, rcs.shape[0], "col")


@ozaki_split_col.register_fake
def _(xw, rcs):
    rp = -(-xw.shape[0] // 128) * 128
    cp = -(-(xw.shape[1] // 2) // 128) * 128
    return xw.new_empty((rcs.shape[0], rp, cp), dtype=torch.bfloat16)


OPS = {
    **{name: _register_gemm(name) for name in _GEMM_NAMES},
    "gemm_lnc_tn": gemm_lnc_tn,
    "syrk": syrk,
    "mp2_energy": mp2_energy,
    "fused_gemm_energy": fused_gemm_energy,
    "batched_pair": batched_pair,
    "j_batched": j_batched,
    "pair_energy_sym": pair_energy_sym,
    "ozaki_gemm": ozaki_gemm,
    "ozaki_emax": ozaki_emax,
    "ozaki_split": ozaki_split,
    "ozaki_emax_col": ozaki_emax_col,
    "ozaki_split_col": ozaki_split_col,
}


def _dtype_checked(name: str, op):
    def checked(*args):
        _check_kernel_operands(name, *args)
        return op(*args)

    checked.__name__ = name
    checked.op = op
    return checked


OPS = {name: _dtype_checked(name, op) for name, op in OPS.items()}
