"""Build `libtrnblas_hip.so` (the gfx950 op library) in-tree.

Every `csrc/*.hip` file is compiled by hipcc for gfx950 only and linked into
one shared library at `trnblas_amd/lib/libtrnblas_hip.so`. The library
exports the C ABI of `include/trnblas_hip.h`; Python loads it with ctypes
(`trnblas_amd/hip/_lib.py`). No CUDA, no HIP/CUDA dual paths.

    python -m trnblas_amd.build          # or trnblas_amd.build.build()
    python -m trnblas_amd.build --asan   # host-side ASan build, lib/asan/
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "lib"
LIBNAME = "libtrnblas_hip.so"
ARCH = "gfx950"

# Packed-fp32 VALU forms (v_pk_*_f32) are disabled for all device code: on
# this fleet some of their forms have given wrong results with no error.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-munsafe-fp-atomics",
    "-Wno-unused-result",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    exe = Path(rocm) / "bin" / "hipcc"
    if exe.exists():
        return str(exe)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return found


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


# Host-side AddressSanitizer (the C-ABI argument checks, error paths and
# drivers; device code is built as usual): each -fsanitize applies to the host
# pass only.
ASAN_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer", "-g"]


def build(verbose: bool = False, jobs: int | None = None, asan: bool = False) -> Path:
    """Compile every HIP source for gfx950 and link the shared library.
    Always rebuilds (this is the build check). Returns the library path.
    asan: a host-ASan build into lib/asan/ instead (load it with
    TRNBLAS_HIP_LIB and the clang ASan runtime preloaded)."""
    libdir = LIBDIR / "asan" if asan else LIBDIR
    libdir.mkdir(parents=True, exist_ok=True)
    objdir = libdir / "obj"
    objdir.mkdir(exist_ok=True)
    cc = hipcc()
    srcs = sources()
    extra = ASAN_FLAGS if asan else []

    def compile_one(src: Path) -> Path:
        obj = objdir / (src.stem + ".o")
        cmd = [cc, *HIPCC_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stderr}")
        return obj

    n = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(n) as ex:
        objs = list(ex.map(compile_one, srcs))
    out = libdir / LIBNAME
    tmp = libdir / (LIBNAME + ".tmp")
    link_extra = ["-Xarch_host", "-fsanitize=address"] if asan else []
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *link_extra, "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv, asan="--asan" in sys.argv)
    print(path)
