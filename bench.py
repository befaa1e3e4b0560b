#!/usr/bin/env python3
"""Benchmark of the hot path on one MI355X: batched JV (C2) + log_sinkhorn (C4).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-sinkhorn]
                    [--no-extra] [--no-cpu-baseline] [--copy-calibration]

Prints ONE JSON line.  ``value`` is the BASELINE metric's lead figure:
batched JV solves/s on C2 = float32 (1024, 64, 64) i.i.d. U[0,1), one step =
one ``torch.ops.assignment.jonker_dense_batch`` call (pre-pass, solve, the
validation readback the op performs), inputs resident in HBM before timing.
The Sinkhorn leg (C4 = (16, 2048, 2048), reg 0.05, 200 iterations) reports
iterations/s and HBM GB/s from the slope between 200- and 20-iteration runs:
one step of this build reads K once (B*N*M*4 algorithmic bytes per
iteration); the rate the reference's two-read formulation would need for the
same iterations/s is reported beside it.  The CPU baseline runs the
reference's own JV solver (oracle/_ref, compiled from its source) or, where
absent, the C restatement, on this host's cores, rank 0 only, on a bounded
sample; Sinkhorn's CPU baseline is the op-for-op torch restatement.
Extra legs (skipped by --no-extra): C3 = JV on (64, 512, 768) with 20% +inf
(solves/s), C5 = unbalanced Sinkhorn on (1, 16384, 16384) (iterations/s,
HBM GB/s) and jonker_compact_batch on the C2 input (solves/s, with the
reference's compact solver as its CPU baseline).  --copy-calibration runs
only a 256 MiB device copy, the known traffic that profiler byte counters
are scaled against.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0  # MI355X published HBM3E bandwidth

# Reduced-cost relaxations c[i][j] - v[j] that the reference algorithm performs
# on the C2 seed-0 batch (all phases, summed over the 1024 problems), counted
# by the instrumented C restatement; tests/test_oracle_jv.py recomputes it.
# Each relaxation touches a cost, a dual and a distance: 12 algorithmic bytes.
JV_C2_RELAXATIONS = 28_681_299
JV_BYTES_PER_RELAXATION = 12

# HBM bytes per launch from rocprofv3 --pmc FETCH_SIZE (x2.00, the factor a
# 256 MiB device copy calibrates) and WRITE_SIZE (x1.00), per dispatch; the
# runs and commands are recorded in profiles/kernels_bench_default.md.
MEASURED_TRAFFIC = {
    # jv_stats_kernel + jv_solve_kernel on C2
    "jv_c2": int(((8244.0 + 8304.0) * 2 + 8.0 + 512.0) * 1024),
    # sk_fused_step + sk_col_merge_blk per C4 iteration: two batch groups of 8,
    # each one pass + one merge (K once, column sums twice)
    "sinkhorn_c4": int(2 * ((66321.6 + 1173.5) * 2 + 2176.0 + 128.0) * 1024),
    # the same pair per C5 iteration (one group)
    "sinkhorn_c5": int(((525986.7 + 8358.5) * 2 + 17530.0 + 128.0) * 1024),
}


def _events_time_ms(fn, steps: int, stream) -> float:
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end)


def bench_jv(steps: int, warmup: int, device) -> dict:
    from torchmatch_amd import _native, workloads

    B, N, M = 1024, 64, 64
    cost_cpu = workloads.jv_uniform(B, N, M, seed=0)
    cost = cost_cpu.to(device)
    op = torch.ops.assignment.jonker_dense_batch
    for _ in range(warmup):
        out = op(cost)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(device)
    t0 = time.perf_counter()
    ms = _events_time_ms(lambda: op(cost), steps, stream)
    wall = time.perf_counter() - t0
    ms_per_step = ms / steps

    # kernel-level: the C-ABI entry launched back to back (no readback)
    lib = _native.lib()
    ws_bytes = lib.tm_jv_workspace_bytes(B, N, M)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    status = torch.zeros(2, dtype=torch.int32, device=device)
    outk = torch.empty(B, N, dtype=torch.int64, device=device)
    sp = stream.cuda_stream

    def launch():
        rc = lib.tm_jv_dense_batch_f32(cost.data_ptr(), B, N, M, outk.data_ptr(),
                                       ws.data_ptr(), ws_bytes, status.data_ptr(), sp)
        if rc != 0:
            raise RuntimeError(f"tm_jv_dense_batch_f32 rc={rc}")

    for _ in range(3):
        launch()
    kreps = max(steps, 20)
    kernel_ms = _events_time_ms(launch, kreps, stream) / kreps
    assert lib.tm_jv_check_status(status.data_ptr(), sp) == 0
    assert torch.equal(outk, out)
    bytes_per_launch = B * N * M * 4 + B * N * 8
    achieved = bytes_per_launch / (kernel_ms * 1e-3) / 1e9
    # LDS roofline of the solve: algorithmic LDS bytes (12 per relaxation) over
    # the launch time, against the measured LDS read peak
    lds_bytes = JV_C2_RELAXATIONS * JV_BYTES_PER_RELAXATION
    lds_achieved = lds_bytes / (kernel_ms * 1e-3) / 1e9
    peak = lds_read_peak(device)
    lds_roofline = {
        "bound": "lds",
        "achieved": round(lds_achieved, 1),
        "peak": round(peak["gbs"], 1) if peak else None,
        "unit": "GB/s",
        "frac": round(lds_achieved / peak["gbs"], 5) if peak else None,
        "algorithmic_bytes": lds_bytes,
        "relaxations_per_solve": round(JV_C2_RELAXATIONS / B, 1),
        "peak_probe": peak["probe"] if peak else "probe library not built",
    }
    return {
        "solves_per_s": B / (ms_per_step * 1e-3),
        "ms_per_step": ms_per_step,
        "wall_s": wall,
        "kernel_ms": kernel_ms,
        "kernel_solves_per_s": B / (kernel_ms * 1e-3),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 3),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 6),
            "traffic": MEASURED_TRAFFIC["jv_c2"],
            "note": "stats pre-pass + LDS-resident solve per launch; the solve is a "
                    "latency-bound sequential chain per problem, HBM is not binding",
        },
        "lds_roofline": lds_roofline,
        "cost_sha256": workloads.sha256(cost_cpu),
        "out": out,
    }


def lds_read_peak(device, iters: int = 4096, reps: int = 5) -> dict | None:
    """LDS read bandwidth of the whole chip (lib/libtm_lds_probe.so): 8
    workgroups of 256 lanes per CU stream conflict-free 16-byte LDS reads."""
    import ctypes

    from torchmatch_amd import _build

    if not _build.PROBE_SO.exists():
        return None
    lib = ctypes.CDLL(str(_build.PROBE_SO))
    lib.tm_probe_lds_read.restype = ctypes.c_int64
    lib.tm_probe_lds_read.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_void_p]
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    blocks = 8 * cus
    sink = torch.zeros(blocks, dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream(device)
    run = lambda: lib.tm_probe_lds_read(sink.data_ptr(), blocks, iters, stream.cuda_stream)
    nbytes = run()
    if nbytes <= 0:
        return None
    best = min(_events_time_ms(run, 1, stream) for _ in range(reps))
    return {"gbs": nbytes / (best * 1e-3) / 1e9, "cus": cus,
            "probe": f"{blocks} workgroups x 256 lanes x {iters} ds_read_b128"}


def bench_sinkhorn(device, n_long: int = 200, n_short: int = 20, reps: int = 3) -> dict:
    from torchmatch_amd import workloads

    B, N, M = 16, 2048, 2048
    reg = 0.05
    cost = workloads.sinkhorn_points(B, N, M, 8, seed=0).to(device)
    a = torch.full((B, N), 1.0 / N, device=device)
    b = torch.full((B, M), 1.0 / M, device=device)
    op = torch.ops.transport.log_sinkhorn
    stream = torch.cuda.current_stream(device)
    op(cost, reg, n_short, a, b)
    torch.cuda.synchronize()

    def best(n_iter):
        times = []
        for _ in range(reps):
            times.append(_events_time_ms(lambda: op(cost, reg, n_iter, a, b), 1, stream))
        return min(times)

    t_long = best(n_long)
    t_short = best(n_short)
    per_iter_ms = (t_long - t_short) / (n_long - n_short)
    return {
        "config": {"workload": "log_sinkhorn C4", "B": B, "N": N, "M": M, "reg": reg,
                   "n_iter": n_long},
        "iters_per_s": 1e3 / per_iter_ms,
        "ms_per_iter": per_iter_ms,
        "op_ms_200_iters": t_long,
        **_sinkhorn_roofline(B, N, M, per_iter_ms, MEASURED_TRAFFIC.get("sinkhorn_c4")),
    }


def _sinkhorn_roofline(B, N, M, per_iter_ms, traffic) -> dict:
    """One step of this build reads K once (row LSE and the column sums come
    from the same registers): B*N*M*4 algorithmic bytes per iteration.  The
    reference's formulation reads K once per half-step; the rate it would need
    for the same iterations/s is reported beside it."""
    one_read = B * N * M * 4
    gbs = one_read / (per_iter_ms * 1e-3) / 1e9
    return {
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "bytes_per_iter": one_read,
            "note": "fused step: one read of K per iteration (+ column partials)",
        },
        "two_pass_equiv_gbs": round(2 * one_read / (per_iter_ms * 1e-3) / 1e9, 1),
    }


def bench_jv_c3(device, reps: int = 3) -> dict:
    """C3: (64, 512, 768) squared distances + jitter, 20% +inf (K = 768 kernel)."""
    from torchmatch_amd import workloads

    cost = workloads.jv_rect_masked().to(device)
    op = torch.ops.assignment.jonker_dense_batch
    op(cost)
    torch.cuda.synchronize()
    ms = _events_time_ms(lambda: op(cost), reps, torch.cuda.current_stream(device)) / reps
    return {"config": {"workload": "jonker_dense_batch C3", "B": 64, "N": 512, "M": 768},
            "solves_per_s": 64 / (ms * 1e-3), "ms_per_batch": ms}


def bench_jv_compact(device, reps: int = 20) -> dict:
    """jonker_compact_batch on the C2 input (1024, 64, 64), op time per batch."""
    from torchmatch_amd import workloads

    cost = workloads.jv_uniform(1024, 64, 64, seed=0).to(device)
    op = torch.ops.assignment.jonker_compact_batch
    for _ in range(3):
        op(cost)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(device)
    ms = sorted(_events_time_ms(lambda: op(cost), 1, stream) for _ in range(reps))[reps // 2]
    return {"config": {"workload": "jonker_compact_batch on C2", "B": 1024, "N": 64, "M": 64},
            "solves_per_s": 1024 / (ms * 1e-3), "ms_per_batch": ms}


def bench_unbalanced_c5(device, n_long: int = 100, n_short: int = 20) -> dict:
    """C5: unbalanced Sinkhorn on (1, 16384, 16384), reg 0.02, rho 1 (slope)."""
    from torchmatch_amd import workloads

    N = 16384
    cost = workloads.sinkhorn_points(1, N, N, 8, seed=0).to(device)
    a = workloads.dirichlet(1, N, 1.0, seed=1).to(device)
    b = workloads.dirichlet(1, N, 1.3, seed=2).to(device)
    op = torch.ops.transport.unbalanced_sinkhorn
    stream = torch.cuda.current_stream(device)
    op(cost, 0.02, n_short, 1.0, a, b)
    torch.cuda.synchronize()
    t_long = min(_events_time_ms(lambda: op(cost, 0.02, n_long, 1.0, a, b), 1, stream)
                 for _ in range(2))
    t_short = min(_events_time_ms(lambda: op(cost, 0.02, n_short, 1.0, a, b), 1, stream)
                  for _ in range(2))
    per_iter_ms = (t_long - t_short) / (n_long - n_short)
    return {"config": {"workload": "unbalanced_sinkhorn C5", "B": 1, "N": N, "M": N,
                       "reg": 0.02, "rho": 1.0},
            "iters_per_s": 1e3 / per_iter_ms, "ms_per_iter": per_iter_ms,
            **_sinkhorn_roofline(1, N, N, per_iter_ms, MEASURED_TRAFFIC.get("sinkhorn_c5"))}


def copy_calibration(device, mib: int = 256, reps: int = 5) -> dict:
    """A plain device copy of known size, for scaling rocprofv3 FETCH/WRITE_SIZE."""
    n = mib * (1 << 20) // 4
    x = torch.rand(n, device=device)
    y = torch.empty_like(x)
    for _ in range(reps):
        y.copy_(x)
    torch.cuda.synchronize()
    return {"copy_bytes_each_way": n * 4, "reps": reps}


def cpu_baseline_jv(budget_s: float = 10.0, compact: bool = False) -> dict:
    from oracle import jv
    from torchmatch_amd import workloads

    cost = workloads.jv_uniform(1024, 64, 64, seed=0).numpy()
    threads = jv.default_threads()
    if jv.ref_available():
        fn, kind = (jv.ref_jv_compact_batch if compact else jv.ref_jv_dense_batch), "reference"
    else:
        fn, kind = (jv.jv_compact_batch if compact else jv.jv_dense_batch), "port"
    fn(cost, threads)  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 5:
        t0 = time.perf_counter()
        fn(cost, threads)
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return {
        "value": 1024 / med,
        "unit": "solves/s",
        "cores": threads,
        "kind": kind,
        "sample": f"C2 (1024,64,64) seed 0, {len(times)} runs over ~{budget_s:.0f}s, median",
    }


def cpu_baseline_sinkhorn(n_iter: int = 3) -> dict:
    from oracle import sinkhorn as sk
    from torchmatch_amd import workloads

    B, N, M = 16, 2048, 2048
    cost = workloads.sinkhorn_points(B, N, M, 8, seed=0)
    a = torch.full((B, N), 1.0 / N)
    t0 = time.perf_counter()
    sk.log_sinkhorn_plan(cost, eps=0.05, n_iter=1, a=a, b=a)
    t1 = time.perf_counter()
    sk.log_sinkhorn_plan(cost, eps=0.05, n_iter=1 + n_iter, a=a, b=a)
    t2 = time.perf_counter()
    per_iter = ((t2 - t1) - (t1 - t0)) / n_iter
    return {
        "value": 1.0 / per_iter if per_iter > 0 else None,
        "unit": "iters/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"C4 (16,2048,2048) reg 0.05, slope of {1 + n_iter} vs 1 iterations",
    }


def main() -> int:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[1])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-sinkhorn", action="store_true")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-extra", action="store_true",
                   help="skip the C3 (K=768 JV) and C5 (unbalanced 16384^2) legs")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only run a 256 MiB device copy (profiler counter calibration)")
    args = p.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (each box has one MI355X); "
              "run with --gpus 1", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py: no ROCm device visible", file=sys.stderr)
        return 2
    import torchmatch_amd  # noqa: F401

    device = torch.device("cuda:0")
    if args.copy_calibration:
        print(json.dumps(copy_calibration(device)), flush=True)
        return 0
    jv_res = bench_jv(args.steps, args.warmup, device)
    line = {
        "metric": "batched JV solves/s (B=1024,N=64) + log_sinkhorn iters/s & HBM GB/s, 1 GPU",
        "value": round(jv_res["solves_per_s"], 1),
        "unit": "solves/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(jv_res["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded torch.rand U[0,1), sha256 "
                + jv_res["cost_sha256"][:16] + ")",
        "config": {"workload": "jonker_dense_batch C2", "B": 1024, "N": 64, "M": 64,
                   "parallelism": "single GPU, one problem per 64-lane workgroup"},
        "kernel": {"ms_per_launch": round(jv_res["kernel_ms"], 5),
                   "solves_per_s": round(jv_res["kernel_solves_per_s"], 1)},
        "roofline": jv_res["roofline"],
        "lds_roofline": jv_res["lds_roofline"],
    }
    if not args.no_sinkhorn:
        sk = bench_sinkhorn(device)
        line["sinkhorn"] = {k: (round(v, 4) if isinstance(v, float) else v)
                            for k, v in sk.items()}
    if not args.no_extra:
        line["jv_c3"] = {k: (round(v, 3) if isinstance(v, float) else v)
                         for k, v in bench_jv_c3(device).items()}
        line["unbalanced_c5"] = {k: (round(v, 4) if isinstance(v, float) else v)
                                 for k, v in bench_unbalanced_c5(device).items()}
        line["jv_compact_c2"] = {k: (round(v, 4) if isinstance(v, float) else v)
                                 for k, v in bench_jv_compact(device).items()}
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_jv()
        if not args.no_extra:
            line["jv_compact_c2"]["cpu_baseline"] = cpu_baseline_jv(5.0, compact=True)
        if not args.no_sinkhorn:
            line["sinkhorn"]["cpu_baseline"] = cpu_baseline_sinkhorn()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
