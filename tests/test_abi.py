"""The C-ABI library loads and exports every entry point of
include/trnblas_hip.h (no GPU needed: no compute call is made)."""

import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "trnblas_hip.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(trnblas_hip_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_surface():
    names = _declared()
    for n in ("trnblas_hip_gemm", "trnblas_hip_syrk", "trnblas_hip_pair_energy",
              "trnblas_hip_ozaki_split", "trnblas_hip_ozaki_gemm", "trnblas_hip_mp2_energy"):
        assert n in names


def test_library_exports_every_declared_symbol():
    from trnblas_amd.hip import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built (run __graft_entry__.build())")
    lib = _lib.load()
    missing = [n for n in _declared() if getattr(lib, n, None) is None]
    assert not missing, missing
    assert set(_declared()) == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"
    assert lib.trnblas_hip_abi_version() == _lib.ABI_VERSION
    assert lib.trnblas_hip_last_error() == b""


def test_argument_errors_are_reported_without_a_gpu():
    # invalid arguments are rejected before any HIP call
    from trnblas_amd.hip import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built")
    lib = _lib.load()
    rc = lib.trnblas_hip_gemm(7, 0, 0, 4, 4, 4, 1.0, None, 4, 0, None, 4, 0, 0.0, None, 4, 0,
                              None, 4, 0, 1, None, 0, None)
    assert rc == _lib.E_ARG and b"dtype" in lib.trnblas_hip_last_error()
    rc = lib.trnblas_hip_pack_k(0, 4, 5, None, 5, 1, 0, None, 4, 20, 1, None)
    assert rc == _lib.E_ARG and b"bad sizes" in lib.trnblas_hip_last_error()  # kp < K
    rc = lib.trnblas_hip_pack_k(1, 4, 5, None, 5, 1, 0, None, 8, 20, 2, None)
    assert rc == _lib.E_ARG and b"batch stride" in lib.trnblas_hip_last_error()
    assert lib.trnblas_hip_pack_k(0, 0, 5, None, 5, 1, 0, None, 8, 0, 1, None) == 0  # R == 0: nothing to do
    rc = lib.trnblas_hip_ozaki_gemm(0, 13, 4, 4, 128, 128, None, 128, 0, None, 128, 0, None,
                                    None, None, 4, 1, None)
    assert rc == _lib.E_ARG and b"slices" in lib.trnblas_hip_last_error()
    assert lib.trnblas_hip_pair_energy_workspace(672, 4656) == (4656 * 28 + 4656) * 8
    # bf16x6: partials (256-byte aligned), then 3 bf16 pieces of every
    # (occupied, virtual) row, virtual rows in pairs, naux rounded up to 64,
    # per operand.
    part = -(-((4656 * 28 + 4656) * 8) // 256) * 256
    pieces = 96 * 672 * 3 * 2304 * 2
    assert lib.trnblas_hip_pair_energy_bf16x6_workspace(672, 2304, 4656, 96, 0) == part + pieces
    odd = -(-(5 * 8 * 3 * 64 * 2) // 256) * 256  # nvir 7 -> 4 row pairs, naux 33 -> 64
    assert lib.trnblas_hip_pair_energy_bf16x6_workspace(7, 33, 3, 5, 5) == 256 + 2 * odd
    # the implicit walk shares one set of pieces (nj == 0) and needs ni >= nocc
    rc = lib.trnblas_hip_pair_energy_bf16x6(7, 33, 16, 2, 231, 16, 0, 231, 33, 16, 16, 16, 3,
                                            6, None, None, None, None, 16, 16, 4096, None)
    assert rc == _lib.E_ARG and b"ni >= nocc" in lib.trnblas_hip_last_error()
    # fp16x3: 2 fp16 pieces per element, then one int32 exponent per
    # (occupied, padded virtual) row, per operand
    pieces2 = 96 * 672 * 2 * 2304 * 2
    exps = -(-(96 * 672 * 4) // 256) * 256
    assert lib.trnblas_hip_pair_energy_fp16x3_workspace(672, 2304, 4656, 96, 0) == part + pieces2 + exps
    odd2 = -(-(5 * 8 * 2 * 64 * 2) // 256) * 256
    exps2 = -(-(5 * 8 * 4) // 256) * 256
    assert lib.trnblas_hip_pair_energy_fp16x3_workspace(7, 33, 3, 5, 5) == 256 + 2 * odd2 + 2 * exps2
    rc = lib.trnblas_hip_pair_energy_fp16x3(7, 33, 16, 2, 231, 16, 0, 231, 33, 16, 16, 16, 3,
                                            6, None, None, None, None, 16, 16, 4096, None)
    assert rc == _lib.E_ARG and b"ni >= nocc" in lib.trnblas_hip_last_error()


def test_syrk_and_triangle_argument_errors_without_a_gpu():
    # the device-decided triangle rule needs its flags when beta != 0, and
    # the triangle check needs an aligned int32[2]; both are refused before
    # any HIP call (the chol_block size bound too)
    import ctypes

    from trnblas_amd.hip import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built")
    lib = _lib.load()
    fake = ctypes.c_void_p(4096)  # never dereferenced: the calls fail their argument checks
    rc = lib.trnblas_hip_syrk_flagged(0, 0, 0, 8, 8, 1.0, fake, 8, 0.5, fake, 8, fake, 8, None,
                                      None, 0, None)
    assert rc == _lib.E_ARG and b"flags" in lib.trnblas_hip_last_error()
    rc = lib.trnblas_hip_triangle_nonzero(0, 8, fake, 8, ctypes.c_void_p(4100), None)
    assert rc == _lib.E_ARG and b"aligned" in lib.trnblas_hip_last_error()
    rc = lib.trnblas_hip_chol_block(129, fake, 129, fake, 129, fake, 0, None)
    assert rc == _lib.E_ARG and b"nb" in lib.trnblas_hip_last_error()
