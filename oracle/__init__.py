"""CPU oracle of the trnblas Level-3 hot path — TEST INFRASTRUCTURE ONLY.

A restatement, in numpy / torch-CPU code of this repository, of the
reference's CPU algorithms for the hot path (trnsci/trnblas 0.13.0), each
function citing the reference file:line it follows:

* `oracle.blas`        gemm / batched_gemm / syrk semantics (trnblas/level3.py)
* `oracle.ozaki`       the Ozaki split, schedule, TwoSum reference and combine
                       (trnblas/ozaki.py)
* `oracle.exact`       the independent near-correctly-rounded fp64 product
                       used to judge gemm_fp64 accuracy (tests/_ozaki_ref.py)
* `oracle.pair_energy` the DF-MP2 pair-energy references
                       (trnblas/nki/dispatch.py, examples/df_mp2.py)
* `oracle.metric`      trsm and the metric factor metric_inv_half
                       (trnblas/level3.py, trnblas/nki/dispatch.py)
* `oracle.df_mp2`      the example's whole DF-MP2 calculation: metric factor,
                       half-transforms, metric contraction, energy
                       (examples/df_mp2.py)

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` may import this package, and only as the checker (or, for
`cpu_baseline`, as the timed stand-in of the reference's CPU path). The
product (`trnblas_amd`) never imports it: the HIP path has no CPU fallback
through the oracle.

How each function is pinned (so that a plausible slip fails a check) is
listed in the header of each module; all functions are pinned — none is
"parity unpinned".
"""
