"""Benchmark of the trnblas Level-3 hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extras]

Headline (one JSON line on stdout): BASELINE.json's metric on its config
`configs[1]`, the fp32 Level-3 mix — one step = SYRK (C = A A^T + 0.5 C on
the lower triangle, A 4096 x 8192) + batched GEMM (64 x (512 x 2048) @
(2048 x 512)) through the public API, inputs resident in HBM. `value` is the
step's algorithmic TFLOP/s (SYRK counted as n (n + 1) k, the triangle).

`roofline` is the dominant kernel of the step (the SYRK kernel): its
algorithmic flops per launch over its average launch time, from HIP events
recorded around every launch of the timed region on the launch stream.
`cpu_baseline` is the reference's CPU path (torch.matmul on the host, the
`_scale_add` epilogue; restated in oracle/blas.py) on the same step.

`extra` carries the other BASELINE configurations: C1 (2048^3 Aᵀ B parity
and time), fp32 GEMM 8192^3 against peak, C3 (the fused DF-MP2 pair energy
against the unfused GPU baseline, with its fp64 energy error), C5 (Ozaki
gemm_fp64 8192^3 against native fp64 DGEMM), and the metric stage
(metric_inv_half and trsm at naux 4096 in fp64 against the host's LAPACK).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

# MI355X published dense peaks (TFLOP/s or TOPS) and HBM bandwidth.
PEAK_FP32_MFMA = 157.3
PEAK_BF16_MFMA = 2500.0
PEAK_FP64_MFMA = 78.6
PEAK_INT8 = 5033.0
PEAK_HBM_GBS = 8000.0

SYRK_N, SYRK_K = 4096, 8192
BATCH, BM, BK, BN = 64, 512, 2048, 512
SYRK_FLOP = SYRK_N * (SYRK_N + 1) * SYRK_K  # triangle count
BATCHED_FLOP = BATCH * 2 * BM * BN * BK
STEP_FLOP = SYRK_FLOP + BATCHED_FLOP
SETTLE_S = 0.3  # untimed steps before the warm-up (clock ramp), seconds of wall time


def committed_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc
    summary (profiles/pmc_traffic.md: FETCH_SIZE + WRITE_SIZE per dispatch,
    scaled by the same counters' reading for a plain copy of known size), or
    None when there is no such summary."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "pmc_traffic.md")
    try:
        for line in open(path):
            if line.startswith(f"traffic_bytes_per_launch[{kernel}]"):
                return float(line.split("=", 1)[1])
    except OSError:
        pass
    return None


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def host_info() -> dict:
    """The host the CPU legs run on: CPU model (lscpu's "Model name", from
    /proc/cpuinfo), the CPUs in this process's affinity mask, P = the
    physical cores among them (distinct (package, core) ids), and
    OMP_WAIT_POLICY."""
    cpus = sorted(os.sched_getaffinity(0))
    model, cores, cur = None, set(), {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" not in line:
                if cur.get("processor") is not None and int(cur["processor"]) in cpus:
                    cores.add((cur.get("physical id"), cur.get("core id")))
                cur = {}
                continue
            k, v = (x.strip() for x in line.split(":", 1))
            cur[k] = v
            if k == "model name" and model is None:
                model = v
        if cur.get("processor") is not None and int(cur["processor"]) in cpus:
            cores.add((cur.get("physical id"), cur.get("core id")))
    except OSError:
        pass
    phys = len(cores) if cores and None not in {c for pair in cores for c in pair} else len(cpus)
    return {"cpu_model": model, "affinity_cpus": len(cpus), "physical_cores_P": phys,
            "omp_wait_policy": os.environ.get("OMP_WAIT_POLICY"),
            "torch_default_threads": torch.get_num_threads()}  # fmt: skip


class threads:
    """torch.set_num_threads(n) for the duration of a block."""

    def __init__(self, n: int):
        self.n = n

    def __enter__(self):
        self.prev = torch.get_num_threads()
        torch.set_num_threads(self.n)

    def __exit__(self, *exc):
        torch.set_num_threads(self.prev)


def cpu_ms(fn, reps: int) -> float:
    """Median wall time of fn() in ms after one untimed call."""
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append((time.perf_counter() - t0) * 1e3)
    return median(ts)


def median(xs):
    xs = sorted(xs)
    return xs[len(xs) // 2]


class LaunchEvents:
    """HIP events around each launch of one kernel (via the kernel-wrapper
    probe), recorded on torch's current stream, i.e. the launch stream."""

    def __init__(self, kernel: str):
        self.kernel, self.pairs, self._open = kernel, [], None

    def __call__(self, kernel, phase):
        if kernel != self.kernel:
            return
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        if phase == "begin":
            self._open = ev
        else:
            self.pairs.append((self._open, ev))

    def mean_ms(self) -> float:
        return sum(a.elapsed_time(b) for a, b in self.pairs) / max(1, len(self.pairs))


def gpu_time_ms(fn, reps: int, warm: int = 1) -> float:
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        torch.cuda.synchronize()
        ts.append(s.elapsed_time(e))
    return median(ts)


def cpu_baseline_level3(A, C, Ab, Bb, n_threads: int) -> dict:
    """The reference's CPU path on one full step (oracle/blas.py), median of 3."""
    from oracle import blas

    Ah, Ch, Abh, Bbh = (x.cpu() for x in (A, C, Ab, Bb))

    def one():
        blas.syrk_cpu(1.0, Ah, 0.5, Ch, uplo="lower")
        blas.batched_gemm_cpu(1.0, Abh, Bbh)

    with threads(n_threads):
        t = cpu_ms(one, 3) * 1e-3
    return {"value": STEP_FLOP / t / 1e12, "unit": "TFLOP/s", "cores": n_threads, "ms": t * 1e3}


def run_extras(dev, tb, only=None, P: int = 1, do_cpu: bool = True) -> dict:
    """The other BASELINE workloads (C1, fp32 8192^3, C3, C5) and the metric
    stage; `only` selects a subset by name. CPU legs run at P threads (the
    physical cores of the affinity mask) and at 2 threads (the reference's
    publishing convention, docs/benchmarks.md:169-173)."""
    from trnblas_amd import df_mp2
    from trnblas_amd.hip import dispatch, kernels

    out = {}
    if only is None or "c1" in only:
        # C1: gemm fp32 A^T B + 0.5 C at 2048^3, against the CPU path
        A, B, C = df_mp2.config1_inputs(dev)

        def pub():
            return tb.gemm(1.0, A, B, beta=0.5, C=C, transA=True)

        def lt():  # hipBLASLt through torch on the same operands (A^T as a view)
            return torch.addmm(C, A.mT, B, beta=0.5)

        # Single calls include the host's time to issue them, so the two are
        # timed in alternating blocks under the same host conditions, and
        # before the CPU legs (whose worker threads compete with the host
        # side of a call while they wind down).
        ts, tls = [], []
        for _ in range(6):
            ts.append(gpu_time_ms(pub, reps=10, warm=5))
            tls.append(gpu_time_ms(lt, reps=10, warm=5))
        t, tl = median(ts), median(tls)
        D = pub()
        Dl = lt()
        # One call between two events includes the host's time to issue it
        # (the public path's routing and argument handling); 20 calls back
        # to back show the GPU time per call, and the launch events bracket
        # the library's kernels alone.
        def b2b(fn, calls=20):
            return gpu_time_ms(lambda: [fn() for _ in range(calls)], reps=5, warm=1) / calls

        t_b2b = b2b(pub)
        tl_b2b = b2b(lt)
        probe = LaunchEvents("gemm")
        kernels._launch_probe = probe
        for _ in range(20):
            tb.gemm(1.0, A, B, beta=0.5, C=C, transA=True)
        kernels._launch_probe = None
        torch.cuda.synchronize()
        tk = probe.mean_ms()
        Ah, Bh, Ch = A.cpu(), B.cpu(), C.cpu()
        from oracle import blas

        with threads(P):
            cpu = blas.gemm_cpu(1.0, Ah, Bh, 0.5, Ch, transA=True)  # the reference's CPU path
            c1_cpu_ms = cpu_ms(lambda: blas.gemm_cpu(1.0, Ah, Bh, 0.5, Ch, transA=True), 5) if do_cpu else None
        with threads(2):
            c1_cpu2_ms = cpu_ms(lambda: blas.gemm_cpu(1.0, Ah, Bh, 0.5, Ch, transA=True), 3) if do_cpu else None
        den = Ah.double().abs().T @ Bh.double().abs() + 0.5 * Ch.double().abs()
        err = float(((D.cpu().double() - cpu.double()) / den).abs().max())
        err_l = float(((Dl.cpu().double() - cpu.double()) / den).abs().max())
        fl = 2 * 2048**3
        out["c1_gemm_2048_transA"] = {
            "ms": t, "tflops": fl / t / 1e9, "frac_fp32_peak": fl / t / 1e9 / PEAK_FP32_MFMA,
            "ms_back_to_back": t_b2b, "tflops_back_to_back": fl / t_b2b / 1e9,
            "kernel_ms": tk, "kernel_tflops": fl / tk / 1e9, "kernel_frac_fp32_peak": fl / tk / 1e9 / PEAK_FP32_MFMA,
            "cw_err_vs_cpu_path": err, "gate": 1e-6, "cpu_ms": c1_cpu_ms, "cpu_threads": P,
            "cpu_ms_at_2_threads": c1_cpu2_ms,
            "route": dispatch._gemm_route(A.mT, B), "torch_hipblaslt_ms": tl,
            "torch_hipblaslt_tflops": fl / tl / 1e9, "torch_hipblaslt_ms_back_to_back": tl_b2b,
            "torch_hipblaslt_cw_err_vs_cpu_path": err_l,
        }  # fmt: skip
        log("c1", out["c1_gemm_2048_transA"])
    if only is None or "gemm8192" in only:
        # fp32 GEMM 8192^3 (north-star target: >= 70 % of fp32 MFMA peak)
        g = torch.Generator().manual_seed(0)
        X = torch.randn(8192, 8192, generator=g).to(dev)
        Y = torch.randn(8192, 8192, generator=g).to(dev)
        t = gpu_time_ms(lambda: tb.gemm(1.0, X, Y), reps=10, warm=2)
        tl = gpu_time_ms(lambda: torch.matmul(X, Y), reps=10, warm=2)
        fl = 2 * 8192**3
        out["gemm_fp32_8192"] = {
            "ms": t, "tflops": fl / t / 1e9, "frac_fp32_peak": fl / t / 1e9 / PEAK_FP32_MFMA,
            "torch_hipblaslt_ms": tl, "torch_tflops": fl / tl / 1e9,
        }  # fmt: skip
        log("gemm8192", out["gemm_fp32_8192"])
        # the same product in bf16 (fp32 accumulate), NN and NT (B^T read in place)
        Xb, Yb = X.bfloat16(), Y.bfloat16()
        del X, Y
        # untimed settle: the first bf16 timing after the fp32 block read
        # ~15 % slow whichever call came first
        gpu_time_ms(lambda: torch.matmul(Xb, Yb), reps=10, warm=5)
        tb_nn = gpu_time_ms(lambda: tb.gemm(1.0, Xb, Yb), reps=10, warm=2)
        tb_nt = gpu_time_ms(lambda: tb.gemm(1.0, Xb, Yb, transB=True), reps=10, warm=2)
        tlb = gpu_time_ms(lambda: torch.matmul(Xb, Yb), reps=10, warm=2)
        tlb_nt = gpu_time_ms(lambda: torch.matmul(Xb, Yb.mT), reps=10, warm=2)
        # the HIP kernel itself (the public call above takes the measured route)
        tk_nn = gpu_time_ms(lambda: kernels.gemm(Xb, Yb, 1.0, 0.0, None), reps=10, warm=2)
        tk_nt = gpu_time_ms(lambda: kernels.gemm(Xb, Yb.mT, 1.0, 0.0, None), reps=10, warm=2)
        out["gemm_bf16_8192"] = {
            # the public call (whichever route it takes) ...
            "public_route_nn": dispatch._gemm_route(Xb, Yb), "public_route_nt": dispatch._gemm_route(Xb, Yb.mT),
            "public_nn_ms": tb_nn, "public_nn_tflops": fl / tb_nn / 1e9,
            "public_nt_ms": tb_nt, "public_nt_tflops": fl / tb_nt / 1e9,
            # ... the hand-written HIP kernel on its own ...
            "kernel_nn_ms": tk_nn, "kernel_nn_tflops": fl / tk_nn / 1e9,
            "kernel_nn_frac_bf16_peak": fl / tk_nn / 1e9 / PEAK_BF16_MFMA,
            "kernel_nt_ms": tk_nt, "kernel_nt_tflops": fl / tk_nt / 1e9,
            "kernel_nt_frac_bf16_peak": fl / tk_nt / 1e9 / PEAK_BF16_MFMA,
            # ... and hipBLASLt (torch.matmul) on its own
            "hipblaslt_nn_ms": tlb, "hipblaslt_nn_tflops": fl / tlb / 1e9,
            "hipblaslt_nn_frac_bf16_peak": fl / tlb / 1e9 / PEAK_BF16_MFMA,
            "hipblaslt_nt_ms": tlb_nt, "hipblaslt_nt_tflops": fl / tlb_nt / 1e9,
            "hipblaslt_nt_frac_bf16_peak": fl / tlb_nt / 1e9 / PEAK_BF16_MFMA,
        }  # fmt: skip
        log("gemm8192bf16", out["gemm_bf16_8192"])
        del Xb, Yb
    if only is None or "c3" in only:
        # C3: fused pair energy vs the unfused GPU baseline (hipBLASLt GEMM + torch),
        # in the three kernel arithmetics (fp16x3 is the default)
        Bp, eo, ev = df_mp2.config3_inputs(dev)
        tf = gpu_time_ms(lambda: kernels.pair_energy_sym(Bp, eo, ev, math="fp16x3"), reps=3, warm=1)
        tb6 = gpu_time_ms(lambda: kernels.pair_energy_sym(Bp, eo, ev, math="bf16x6"), reps=3, warm=1)
        tf32 = gpu_time_ms(lambda: kernels.pair_energy_sym(Bp, eo, ev, math="fp32"), reps=3, warm=1)
        tu = gpu_time_ms(lambda: dispatch._torch_chunked_pair_energy(Bp, eo, ev), reps=3, warm=1)
        e_hip = float(kernels.pair_energy_sym(Bp, eo, ev, math="fp16x3"))
        e_b6 = float(kernels.pair_energy_sym(Bp, eo, ev, math="bf16x6"))
        e_f32 = float(kernels.pair_energy_sym(Bp, eo, ev, math="fp32"))
        e_unf = float(dispatch._torch_chunked_pair_energy(Bp, eo, ev))
        Bd, eod, evd = Bp.double(), eo.double(), ev.double()
        e64 = torch.zeros((), dtype=torch.float64, device=dev)
        for i in range(Bp.shape[0]):
            T = torch.matmul(Bd[i].unsqueeze(0), Bd[i:].transpose(1, 2))
            Dn = eod[i] + eod[i:, None, None] - evd[None, :, None] - evd[None, None, :]
            e = (T * (2.0 * T - T.transpose(1, 2)) / Dn).sum(dim=(1, 2))
            w = torch.full_like(e, 2.0)
            w[0] = 1.0
            e64 += (w * e).sum()
        e64 = float(e64)
        del Bd
        fl = 96 * 97 / 2 * 2 * 672 * 672 * 2304
        # the fused entry point's launches (split + fused kernel + sums), timed
        # with HIP events on the launch stream
        probe = LaunchEvents("pair_energy")
        kernels._launch_probe = probe
        for _ in range(3):
            kernels.pair_energy_sym(Bp, eo, ev, math="fp16x3")
        kernels._launch_probe = None
        torch.cuda.synchronize()
        t_launch = probe.mean_ms()
        roof = {
            "kernel": "split_f16x3_kernel + pair_energy_quad_kernel "
                      "(trnblas_hip_pair_energy_fp16x3)",
            "bound": "mfma", "launch_ms": t_launch,
            "achieved": 3 * fl / t_launch / 1e9, "peak": PEAK_BF16_MFMA, "unit": "TFLOP/s (f16 MFMA)",
            "frac": 3 * fl / t_launch / 1e9 / PEAK_BF16_MFMA,
            "achieved_fp32_equiv": fl / t_launch / 1e9, "ceiling_fp32_equiv": PEAK_BF16_MFMA / 3,
            "algorithmic_flop_per_launch": fl, "traffic": committed_traffic("pair_energy_quad"),
        }  # fmt: skip
        # The reference's CPU path (the fp32 torch pair loop of
        # dispatch.py:2514-2533, restated in oracle/pair_energy.py) over all
        # 9216 ordered pairs, once.
        from oracle import pair_energy as pe

        Bh, eoh, evh = Bp.cpu(), eo.cpu(), ev.cpu()
        e_cpu, cpu_loop_ms, cpu2_sample_ms = float("nan"), None, None
        if do_cpu:
            with threads(P):
                t0 = time.perf_counter()
                e_cpu = float(pe.batched_pair_cpu(Bh, eoh, evh))
                cpu_loop_ms = (time.perf_counter() - t0) * 1e3
            # at 2 threads a bounded sample: rows i = 0..11 (1152 of the 9216
            # ordered pairs, 1/8 of the loop), scaled by 8
            with threads(2):
                t0 = time.perf_counter()
                pe.batched_pair_cpu(Bh, eoh, evh, rows=range(12))
                cpu2_sample_ms = (time.perf_counter() - t0) * 1e3
        del Bh
        out["pair_energy_c3_96_672_2304"] = {
            "fused_ms": tf, "fused_math": "fp16x3", "unfused_gpu_ms": tu,
            "speedup_vs_unfused": tu / tf, "tflops_sym": fl / tf / 1e9,
            "f16_mfma_tflops": 3 * fl / tf / 1e9,
            "frac_f16_peak": 3 * fl / tf / 1e9 / PEAK_BF16_MFMA,
            "energy_fp64": e64, "rel_err_fused_vs_fp64": abs(e_hip - e64) / abs(e64),
            "fused_bf16x6_ms": tb6, "speedup_bf16x6_vs_unfused": tu / tb6,
            "frac_bf16_peak_bf16x6": 6 * fl / tb6 / 1e9 / PEAK_BF16_MFMA,
            "rel_err_fused_bf16x6_vs_fp64": abs(e_b6 - e64) / abs(e64),
            "fused_fp32_mfma_ms": tf32, "speedup_fp32_mfma_vs_unfused": tu / tf32,
            "frac_fp32_peak_fp32_mfma": fl / tf32 / 1e9 / PEAK_FP32_MFMA,
            "rel_err_fused_fp32_mfma_vs_fp64": abs(e_f32 - e64) / abs(e64),
            "rel_err_unfused_fp32_vs_fp64": abs(e_unf - e64) / abs(e64), "gate": 1e-6,
            "cpu_fp32_loop_ms": cpu_loop_ms, "rel_err_cpu_fp32_loop_vs_fp64": abs(e_cpu - e64) / abs(e64),
            "cpu_sample": "the whole fp32 torch pair loop (9216 ordered pairs), once, at P threads",
            "cpu_threads": P,
            "cpu_fp32_loop_ms_at_2_threads": None if cpu2_sample_ms is None else 8 * cpu2_sample_ms,
            "cpu_sample_at_2_threads": "rows i = 0..11 of the loop (1152 ordered pairs), once, x8",
            "roofline": roof,
        }  # fmt: skip
        log("c3", out["pair_energy_c3_96_672_2304"])
        del Bp
    if only is None or "c4" in only:
        # C4: the DF-MP2 chain at its real size (nao 1024, nocc 256, nvir 768,
        # naux 4096): two half-transform batched GEMMs into B, then the fused
        # pair energy (fp16x3); 1.63e14 algorithmic flop (i <= j pair count)
        nao, nocc, nvir, naux = 1024, 256, 768, 4096
        eri, Co, Cv, eo4, ev4 = df_mp2.chain_inputs(nao, nocc, nvir, naux, dev, seed=4)
        th = gpu_time_ms(lambda: df_mp2.half_transform(eri, Co, Cv), reps=3, warm=1)
        B4 = df_mp2.half_transform(eri, Co, Cv)
        del eri
        te = gpu_time_ms(lambda: kernels.pair_energy_sym(B4, eo4, ev4, math="fp16x3"), reps=2, warm=1)
        e4 = float(kernels.pair_energy_sym(B4, eo4, ev4, math="fp16x3"))
        fl = df_mp2.chain_flops(nao, nocc, nvir, naux)
        tot = fl["half1"] + fl["half2"] + fl["energy"]
        t_all = th + te
        out["df_mp2_chain_c4_1024_256_768_4096"] = {
            "half_transform_ms": th, "energy_ms": te, "chain_ms": t_all, "energy": e4,
            "flop": tot, "tflops": tot / t_all / 1e9,
            "half_transform_tflops": (fl["half1"] + fl["half2"]) / th / 1e9,
            "energy_tflops_sym": fl["energy"] / te / 1e9, "energy_math": "fp16x3",
            "half_transform_frac_fp32_peak": (fl["half1"] + fl["half2"]) / th / 1e9 / PEAK_FP32_MFMA,
            "energy_frac_f16_peak": 3 * fl["energy"] / te / 1e9 / PEAK_BF16_MFMA,
            "parity": "tests/test_config4_gpu.py: rel <= 1e-6 against the fp64 chain on the device",
        }  # fmt: skip
        log("c4", out["df_mp2_chain_c4_1024_256_768_4096"])
        del B4
        torch.cuda.empty_cache()
    if only is None or "c5" in only:
        # C5: Ozaki gemm_fp64 at 8192^3, k = 8, against native fp64 DGEMM
        n = 8192
        Ao, Bo = df_mp2.config5_inputs(dev, n, seed=5)
        to = gpu_time_ms(lambda: tb.gemm_fp64(Ao, Bo, mode="fast"), reps=3, warm=1)
        tx = gpu_time_ms(lambda: tb.gemm_fp64(Ao, Bo, mode="exact"), reps=3, warm=1)
        td = gpu_time_ms(lambda: torch.matmul(Ao, Bo), reps=3, warm=1)
        Cd = Ao @ Bo
        den = Ao.abs() @ Bo.abs()
        err = float(((tb.gemm_fp64(Ao, Bo, mode="fast") - Cd).abs() / den).max())
        errx = float(((tb.gemm_fp64(Ao, Bo, mode="exact") - Cd).abs() / den).max())
        ops = 36 * 2 * n**3
        # slice counts 8..12 (fast mode): time and max |C - DGEMM| / (|A||B|);
        # the difference to DGEMM settles at DGEMM's own error once the
        # truncation is below it (tests/test_config5_slices_gpu.py judges each
        # k against a near-exact product over the whole output: k = 11 is the
        # smallest that meets the reference's host gate on this data)
        sweep = []
        for k in range(8, 13):
            tk = gpu_time_ms(lambda: tb.gemm_fp64(Ao, Bo, slices=k, mode="fast"), reps=3, warm=1)
            ek = float(((tb.gemm_fp64(Ao, Bo, slices=k, mode="fast") - Cd).abs() / den).max())
            opk = k * (k + 1) // 2 * 2 * n**3
            sweep.append({
                "k": k, "ms": tk, "int8_tops": opk / tk / 1e9, "frac_int8_peak": opk / tk / 1e9 / PEAK_INT8,
                "fp64_equiv_tflops": 2 * n**3 / tk / 1e9, "max_cw_diff_vs_dgemm": ek,
            })  # fmt: skip
        # the reference's gemm_fp64 off the device: host fp64 A @ B
        # (nki/dispatch.py:965-966), the whole product at P threads, and at 2
        # threads a bounded sample (rows 0..1023, 1/8 of the work) x8
        c5_cpu = {}
        if do_cpu:
            Ah, Bh = Ao.cpu(), Bo.cpu()
            with threads(P):
                t0 = time.perf_counter()
                Ah @ Bh
                c5_cpu["host_fp64_ms"] = (time.perf_counter() - t0) * 1e3
            with threads(2):
                t0 = time.perf_counter()
                Ah[:1024] @ Bh
                c5_cpu["host_fp64_ms_at_2_threads"] = 8 * (time.perf_counter() - t0) * 1e3
            c5_cpu.update(host_threads=P, host_sample_at_2_threads="rows 0..1023 of A @ B, once, x8")
            del Ah, Bh
        # scheme II (mode "crt": one int8 GEMM per Chinese-remainder modulus)
        from trnblas_amd.hip import kernels as _k

        crt_sweep = []
        for k in range(8, 13):
            tk = gpu_time_ms(lambda: tb.gemm_fp64(Ao, Bo, slices=k, mode="crt"), reps=3, warm=1)
            ek = float(((tb.gemm_fp64(Ao, Bo, slices=k, mode="crt") - Cd).abs() / den).max())
            nm = _k.crt_moduli(k, n)
            opk = nm * 2 * n**3
            crt_sweep.append({
                "k": k, "moduli": nm, "ms": tk, "int8_tops": opk / tk / 1e9,
                "frac_int8_peak": opk / tk / 1e9 / PEAK_INT8, "fp64_equiv_tflops": 2 * n**3 / tk / 1e9,
                "max_cw_diff_vs_dgemm": ek,
            })  # fmt: skip
        # the smallest slice counts that meet the reference's host gate over the
        # whole output on this data (asserted by tests/test_config5_slices_gpu.py)
        k_host, k_host_crt = 11, 10
        t_host = next(x["ms"] for x in sweep if x["k"] == k_host)
        t_host_crt = next(x["ms"] for x in crt_sweep if x["k"] == k_host_crt)
        out["ozaki_gemm_fp64_c5_8192_k8"] = {
            "ms": to, "mode": "fast (default: int32 diagonals, fp64 recombination)",
            "int8_tops": ops / to / 1e9, "frac_int8_peak": ops / to / 1e9 / PEAK_INT8,
            "fp64_equiv_tflops": 2 * n**3 / to / 1e9, "native_dgemm_ms": td,
            "native_dgemm_tflops": 2 * n**3 / td / 1e9, "max_cw_err_vs_dgemm": err,
            "exact_mode_ms": tx, "exact_mode_frac_int8_peak": ops / tx / 1e9 / PEAK_INT8,
            "exact_mode_max_cw_err_vs_dgemm": errx, "slice_sweep_fast": sweep,
            "slice_sweep_crt": crt_sweep,
            "host_accurate": {
                "gate": "max(4 host, 4e-15) over the whole output, asserted: tests/test_config5_slices_gpu.py",
                "native_dgemm_ms": td,
                "fast": {"slices": k_host, "ms": t_host, "fp64_equiv_tflops": 2 * n**3 / t_host / 1e9,
                         "speedup_vs_dgemm": td / t_host},
                "crt": {"slices": k_host_crt, "ms": t_host_crt,
                        "fp64_equiv_tflops": 2 * n**3 / t_host_crt / 1e9, "speedup_vs_dgemm": td / t_host_crt},
            },
            **c5_cpu,
            "accuracy_gate": "every element within the 8-slice error bound (C5 wide-range data): "
            "tests/test_api_gpu.py::test_config5_gemm_fp64_accuracy_full_size, both modes",
        }  # fmt: skip
        log("c5", out["ozaki_gemm_fp64_c5_8192_k8"])
    if only is None or "metric" in only:
        # metric stage at C4's naux = 4096: J^-1/2 as the inverse Cholesky
        # factor, and one trsm with naux right-hand sides, in fp64 on the
        # device against the host's LAPACK
        n = 4096
        g = torch.Generator().manual_seed(7)
        S = torch.randn(n, n, generator=g, dtype=torch.float64)
        Jh = S @ S.T / n + torch.eye(n, dtype=torch.float64)
        J = Jh.to(dev)
        tm = gpu_time_ms(lambda: tb.metric_inv_half(J), reps=5, warm=2)
        X = tb.metric_inv_half(J)
        resid = float((X.T @ J @ X - torch.eye(n, device=dev, dtype=torch.float64)).abs().max())
        L = torch.linalg.cholesky(J)
        R = torch.randn(n, n, generator=g, dtype=torch.float64).to(dev)
        tt = gpu_time_ms(lambda: tb.trsm(1.0, L, R, side="left", uplo="lower"), reps=5, warm=2)
        Y = tb.trsm(1.0, L, R, side="left", uplo="lower")
        tres = float(((L @ Y - R).abs().max() / R.abs().max()))
        t0 = time.perf_counter()
        Lh = torch.linalg.cholesky(Jh)
        torch.linalg.solve_triangular(Lh.mT, torch.eye(n, dtype=torch.float64), upper=True)
        lapack_ms = (time.perf_counter() - t0) * 1e3
        fl = 2 * n**3 / 3  # algorithmic: Cholesky n^3 / 3 + triangular inverse n^3 / 3
        out["metric_inv_half_fp64_4096"] = {
            "ms": tm, "tflops": fl / tm / 1e9, "frac_fp64_peak": fl / tm / 1e9 / PEAK_FP64_MFMA,
            "max_abs_XtJX_minus_I": resid, "trsm_4096x4096_ms": tt,
            "trsm_tflops": n**3 / tt / 1e9, "trsm_rel_residual": tres,
            "cpu_lapack_ms": lapack_ms, "cpu_threads": torch.get_num_threads(),
        }  # fmt: skip
        log("metric", out["metric_inv_half_fp64_4096"])
        del J, L, R, X, Y
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default=None,
                    help="comma-separated subset of the extra workloads: c1,gemm8192,c3,c4,c5,metric")
    ap.add_argument(
        "--calibrate-copy",
        action="store_true",
        help="also run a plain 256 MiB device copy (the reference kernel for rocprofv3 "
        "FETCH_SIZE / WRITE_SIZE scaling)",
    )
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(
            "bench.py measures one MI355X: the hot path is single-GPU in this build "
            f"(asked for --gpus {args.gpus}, WORLD_SIZE {world}); run with --gpus 1.",
            file=sys.stderr,
        )
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        sys.exit(2)
    import trnblas_amd as tb
    from trnblas_amd import df_mp2
    from trnblas_amd.hip import dispatch, kernels

    dispatch._REQUIRE_HIP = True  # a kernel error fails the bench, never falls back
    dev = torch.device("cuda", 0)
    A, C, Ab, Bb = df_mp2.config2_inputs(dev)

    def step():
        S = tb.syrk(1.0, A, beta=0.5, C=C, uplo="lower")
        D = tb.batched_gemm(1.0, Ab, Bb)
        return S, D

    # Clock settle: after an idle spell the GPU's clocks ramp up over ~50 ms
    # of this step (the SYRK launch falls from 1.26 to 1.10 ms, then stays);
    # steps run untimed for SETTLE_S seconds of wall time first, then the W
    # warm-up steps, so the timed steps see the steady clocks at any --warmup.
    t_settle = time.perf_counter()
    settle_steps = 0
    while time.perf_counter() - t_settle < SETTLE_S:
        for _ in range(5):
            step()
        torch.cuda.synchronize()
        settle_steps += 5
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    probe = LaunchEvents("syrk")
    kernels._launch_probe = probe
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kernels._launch_probe = None
    ms_per_step = wall / args.steps * 1e3
    value = STEP_FLOP / (wall / args.steps) / 1e12
    syrk_ms = probe.mean_ms()
    achieved = SYRK_FLOP / (syrk_ms * 1e-3) / 1e12
    roofline = {
        "kernel": "gemm_dma_kernel<float, true, true, SYRK> (trnblas_hip_syrk)",
        "bound": "mfma",
        "achieved": achieved,
        "peak": PEAK_FP32_MFMA,
        "unit": "TFLOP/s",
        "frac": achieved / PEAK_FP32_MFMA,
        "traffic": committed_traffic("syrk"),
        "launch_ms": syrk_ms,
        "launches": len(probe.pairs),
        "algorithmic_flop_per_launch": SYRK_FLOP,
    }
    if args.calibrate_copy:
        src = torch.empty(64 << 20, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    # parity of the timed step (the outputs the step produced)
    S, D = step()
    torch.cuda.synchronize()
    Ad = A.double()
    ref = Ad @ Ad.T + 0.5 * (torch.tril(C.double()) + torch.tril(C.double(), -1).T)
    den = Ad.abs() @ Ad.abs().T + 0.5 * C.double().abs()
    syrk_err = float(((S.double() - ref) / den).abs().max())
    refb = Ab.double() @ Bb.double()
    denb = Ab.double().abs() @ Bb.double().abs()
    bat_err = float(((D.double() - refb) / denb).abs().max())
    del ref, den, refb, denb, Ad
    t_b = gpu_time_ms(lambda: tb.batched_gemm(1.0, Ab, Bb), reps=20, warm=20)  # past the clock ramp
    cpu = None
    host = host_info()
    P = host["physical_cores_P"]
    if not args.no_cpu:
        cpu = cpu_baseline_level3(A, C, Ab, Bb, P)
        cpu2 = cpu_baseline_level3(A, C, Ab, Bb, 2)
        cpu.update(kind="port", sample="one full step (C2a SYRK + C2b batched), median of 3",
                   at_2_threads=cpu2["value"], ms_at_2_threads=cpu2["ms"], host=host)  # fmt: skip
    extra = {
        "syrk_c2a": {"ms": syrk_ms, "tflops_triangle": achieved, "cw_err_vs_fp64": syrk_err},
        "batched_c2b": {"ms": t_b, "tflops": BATCHED_FLOP / t_b / 1e9, "cw_err_vs_fp64": bat_err},
    }
    if not args.no_extras:
        only = None if args.only is None else set(args.only.split(","))
        extra.update(run_extras(dev, tb, only, P=P, do_cpu=not args.no_cpu))
    line = {
        "metric": "GEMM TFLOP/s & %MFMA peak; DF-MP2 pair-energy ms at 96/672/2304",
        "value": value,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle": {"seconds": SETTLE_S, "steps": settle_steps},
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1), BASELINE.json configs)",
        "config": {
            "workload": "configs[1] Level-3 mix fp32: syrk lower 4096x8192 + batched_gemm 64x512x2048x512",
            "syrk": [SYRK_N, SYRK_K],
            "batched": [BATCH, BM, BK, BN],
            "step_flop": STEP_FLOP,
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
