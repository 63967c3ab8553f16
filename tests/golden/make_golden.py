"""Write the Ozaki golden vectors from the reference itself (build container
only; /root/reference does not exist on the GPU box).

Loads the reference's trnblas/ozaki.py as a standalone module (it needs only
numpy and torch) and records, for small seeded inputs: the digits and
exponents of `split` (per row and per column, extreme / zero / subnormal
rows, the two-factor scaling), the (hi, lo) of `reference_from_digits`, and
the fp64 result of `reference_gemm` (including the narrow-N swap, K >= 4096
group cuts and multi-pair groups). These are the functions whose bitwise
output no closed form pins; everything else is pinned by invariants and
closed forms in the tests.

    python tests/golden/make_golden.py      # writes tests/golden/ozaki_golden.npz
"""

import importlib.util
import os
import sys

import numpy as np
import torch

REF = "/root/reference/trnblas/ozaki.py"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ozaki_golden.npz")


def load_reference():
    spec = importlib.util.spec_from_file_location("reference_ozaki", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def split_matrix():
    X = np.zeros((12, 70))
    rng = np.random.default_rng(20)
    X[0] = np.linspace(-1e300, 1e300, 70)
    X[1] = np.linspace(-1e-300, 1e-300, 70)
    X[2, 5] = 5e-324
    X[4] = rng.standard_normal(70) * 10.0 ** rng.uniform(-40, 40, 70)
    X[5] = rng.standard_normal(70)
    X[6] = (rng.integers(-(2**20), 2**20, 70) + rng.choice([0.0, 0.5, -0.5], 70)) * 2.0**-63
    X[6, 0] = 1.0 - 2.0**-52  # ties on the digit grid
    X[7:] = rng.standard_normal((5, 70)) * 1e3
    X[7, 3] = 0.0
    return X


def main():
    oz = load_reference()
    data = {}
    X = split_matrix()
    data["split_X"] = X
    for per in ("row", "col"):
        for k in (1, 8, 12):
            d, e = oz.split(torch.from_numpy(X), k, per=per, pad=(1, 1))
            data[f"split_{per}_k{k}_d"] = d.to(torch.float32).numpy().astype(np.int8)
            data[f"split_{per}_k{k}_e"] = e.astype(np.int64)
    # reference_gemm cases: (M, K, N, k, dist, seed)
    cases = [
        (24, 300, 17, 8, "normal", 1),  # kt = 3 < 32: multi-pair groups
        (5, 4100, 3, 8, "normal", 2),  # narrow N < 512 < ... swap; kt = 33: cut groups
        (10, 200, 12, 10, "logu4", 3),  # wide range, k = 10
        (7, 129, 9, 3, "normal", 4),  # Kp = 256, kt = 2
        (16, 64, 600, 12, "normal", 5),  # N >= 512: no swap, k = 12
    ]
    for c, (M, K, N, k, dist, seed) in enumerate(cases):
        rng = np.random.default_rng(seed)
        if dist == "normal":
            A, B = rng.standard_normal((M, K)), rng.standard_normal((K, N))
        else:
            A = rng.standard_normal((M, K)) * 10.0 ** rng.uniform(-4, 4, (M, K))
            B = rng.standard_normal((K, N)) * 10.0 ** rng.uniform(-4, 4, (K, N))
        C = oz.reference_gemm(torch.from_numpy(A), torch.from_numpy(B), k).numpy()
        data[f"gemm{c}_A"], data[f"gemm{c}_B"], data[f"gemm{c}_C"] = A, B, C
        data[f"gemm{c}_k"] = np.array(k)
        if c == 0:  # the raw (hi, lo) of the kernel model, unswapped
            da = oz.split_a(torch.from_numpy(A), k)
            db = oz.split_b(torch.from_numpy(B), k)
            at = oz.kmajor(da.d, da.kmajor)
            bt = oz.kmajor(db.d, db.kmajor)
            data["gemm0_hilo"] = oz.reference_from_digits(at, bt[:, :, :N])
    sch = oz.schedule(4, 3)
    data["schedule_4_3_scales"] = np.array([s for _, s, _ in sch])
    data["n_products_8"] = np.array(oz.n_products(8))
    data["exponent_offset_8"] = np.array(oz.exponent_offset(8))
    np.savez_compressed(OUT, **data)
    print(OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    sys.exit(main())
