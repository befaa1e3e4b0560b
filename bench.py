#!/usr/bin/env python3
"""Benchmark of the hot path on one MI355X: batched JV (C2) + log_sinkhorn (C4).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-sinkhorn]
                    [--no-extra] [--no-cpu-baseline] [--copy-calibration]
                    [--no-host-facts]

Prints ONE JSON line.  ``value`` is the BASELINE metric's lead figure:
batched JV solves/s on C2 = float32 (1024, 64, 64) i.i.d. U[0,1), one step =
one ``torch.ops.assignment.jonker_dense_batch`` call (the solve launch, which
also takes the batch statistics, and the wait for its validated result that
the op performs), inputs resident in HBM before timing.  The Sinkhorn leg (C4 = (16, 2048, 2048), reg 0.05, 200 iterations)
reports iterations/s and HBM GB/s from the slope between 200- and
20-iteration runs; one step of this build reads K once (B*N*M*4 algorithmic
bytes per iteration).  Beside it, the same kernel shape at B = 64 (1 GiB of
K, four times the 256 MB Infinity Cache) shows the rate without cache
residency.

The JV leg also times the op on 16 seeds of the C2 shape (p50 / p90 / max):
a batch holding a problem that fails the certificate pays its exact replay.

CPU baselines run on this host's cores, rank 0 only, on bounded samples: JV
(C1, C2 on all threads and on one thread, C3, the compact solver) on the
reference's own solver compiled from its source (oracle/_ref) or, where
absent, the C restatement; Sinkhorn on the op-for-op torch restatement, C4
for its full 200 iterations and C5 for 20.  Extra legs (skipped by
--no-extra): C3 = JV on (64, 512, 768) with 20% +inf, C5 = unbalanced
Sinkhorn on (1, 16384, 16384), jonker_compact_batch on the C2 input and C1 =
JV on (8, 16, 16).  --copy-calibration runs only a 256 MiB
device copy, the known traffic that profiler byte counters are scaled
against.  ``host`` records the CPU model, core counts and versions;
``inputs`` the seed and sha256 of every input.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import subprocess
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

# The device kernel's certified path on the C2 seed-0 batch: its slowest
# problem (456) takes 314 sequential steps (rows scanned + paths) in the
# shortest-path searches, each needing one wave-wide argmin before the next
# (oracle.jv.sap_batch_counted; tests/test_oracle_jv.py recomputes it).
JV_C2_CRITICAL_STEPS = 314
# C3 seed 0: the reference order's sequential steps on its slowest problem
# (problem 16: 2,496 augmenting row reduction steps + 254 paths + 0 scanned
# rows; oracle.jv.jv_dense_batch_steps, recomputed by tests/test_oracle_jv.py).
# The K = 768 kernel replays that order, one step after another.
JV_C3_CRITICAL_STEPS = 2750

# HBM bytes per launch from rocprofv3 --pmc FETCH_SIZE (x2.00, the factor a
# 256 MiB device copy calibrates) and WRITE_SIZE (x1.00), per dispatch; the
# runs and commands are recorded in the profiles/ summaries.
MEASURED_TRAFFIC = {
    # the fused solve launch on C2 (the op's only launch on this batch)
    "jv_c2": int((8342.0 * 2 + 584.0) * 1024),
    # the K = 768 solve launch on C3 (its tile rows mostly from L2 / MALL)
    "jv_c3": int((2151.0 * 2 + 256.0) * 1024),
    # sk_fused_step + sk_col_merge_blk per C4 iteration: two batch groups of 8,
    # each one pass + one merge (K once, column sums twice)
    "sinkhorn_c4": int(2 * ((66378.0 + 1243.0) * 2 + 2369.1 + 320.0) * 1024),
    # the same per iteration of the B = 64 control (two groups of 32; K read
    # with non-temporal loads)
    "sinkhorn_b64": int(2 * ((267124.2 + 1771.0) * 2 + 3328.0 + 1280.0) * 1024),
    # the same pair per C5 iteration (one group)
    "sinkhorn_c5": int(((533822.9 + 8411.5) * 2 + 18453.4 + 320.0) * 1024),
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


def _probe_lib():
    from torchmatch_amd import _build

    if not _build.PROBE_SO.exists():
        return None
    lib = ctypes.CDLL(str(_build.PROBE_SO))
    lib.tm_probe_lds_read.restype = ctypes.c_int64
    lib.tm_probe_lds_read.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_void_p]
    lib.tm_probe_argmin_chain.restype = ctypes.c_int
    lib.tm_probe_argmin_chain.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                          ctypes.c_void_p]
    lib.tm_probe_hbm_read.restype = ctypes.c_int64
    lib.tm_probe_hbm_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                      ctypes.c_int, ctypes.c_void_p]
    return lib


def hbm_read_ceiling(buf: torch.Tensor, blocks: int = 4096, reps: int = 5) -> dict | None:
    """What one kernel that reads `buf` once reaches (bench_probes.so: 4096
    workgroups, each a contiguous range, eight 16-byte non-temporal loads per
    lane in flight), best of `reps`: the practical ceiling of a read-once pass
    on this chip, beside the 8 TB/s published peak."""
    lib = _probe_lib()
    if lib is None:
        return None
    sink = torch.zeros(blocks, dtype=torch.float32, device=buf.device)
    stream = torch.cuda.current_stream(buf.device)
    nbytes = buf.numel() * buf.element_size()
    run = lambda: lib.tm_probe_hbm_read(buf.data_ptr(), nbytes, sink.data_ptr(), blocks,
                                        stream.cuda_stream)
    if run() != nbytes:
        return None
    torch.cuda.synchronize()
    best = min(_events_time_ms(run, 1, stream) for _ in range(reps))
    return {"gbs": round(nbytes / (best * 1e-3) / 1e9, 1), "bytes": nbytes,
            "probe": f"{blocks} workgroups x 256 lanes, contiguous ranges, 8 x 16 B "
                     "non-temporal loads in flight per lane, best of 5"}


def lds_read_peak(device, iters: int = 4096, reps: int = 5) -> dict | None:
    """LDS read bandwidth of the whole chip (bench_probes.so): 8 workgroups
    of 256 lanes per CU stream conflict-free 16-byte LDS reads."""
    lib = _probe_lib()
    if lib is None:
        return None
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


def argmin_chain(device, iters: int = 20000) -> dict | None:
    """Cycles per dependent wave-wide (minimum, argmin lane) round and the
    shader clock, from one wave (bench_probes.so)."""
    lib = _probe_lib()
    if lib is None:
        return None
    x = torch.rand(64, device=device)
    out = torch.zeros(3, dtype=torch.int64, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    best = None
    for _ in range(3):
        if lib.tm_probe_argmin_chain(x.data_ptr(), out.data_ptr(), iters, stream) != 0:
            return None
        cycles, ticks = (int(v) for v in out[:2].cpu())
        if best is None or cycles < best[0]:
            best = (cycles, ticks)
    cycles, ticks = best
    return {"cycles_per_round": cycles / iters, "clock_ghz": cycles / (ticks * 10.0)}


def bench_jv(steps: int, warmup: int, device) -> dict:
    from torchmatch_amd import _native
    import workloads

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

    # kernel-level: the asynchronous C-ABI entry launched back to back, timed
    # with one pair of events on the launch stream over the repeats (an event
    # pair around a single launch adds 4-6 us on this platform): the fused
    # solve plus the finishing launch the asynchronous entry always issues
    # (the op itself, which waits on the host, runs the solve alone on this
    # batch); the profiler's durations of jv_solve_kernel<false, 1> and
    # <false, 2> add up to it
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
    replays = ctypes.c_uint32(0)
    lib.tm_jv_read_replays(ctypes.c_void_p(ws.data_ptr()), ctypes.byref(replays),
                           ctypes.c_void_p(sp))

    bytes_per_launch = B * N * M * 4 + B * N * 8
    achieved = bytes_per_launch / (kernel_ms * 1e-3) / 1e9
    # LDS, as an equivalent rate: the reference algorithm's LDS bytes (12 per
    # relaxation c[i][j] - v[j]) over this kernel's launch time, against the
    # measured LDS read peak.  The certified path does not perform those
    # relaxations (it issues a few hundred LDS instructions per problem), so
    # this prices the work in the reference's units, not traffic the kernel
    # makes.
    lds_bytes = JV_C2_RELAXATIONS * JV_BYTES_PER_RELAXATION
    lds_achieved = lds_bytes / (kernel_ms * 1e-3) / 1e9
    peak = lds_read_peak(device)
    lds_roofline = {
        "bound": "lds",
        "binding": False,
        "kind": "equivalent rate (reference algorithm's relaxations x 12 B / this launch)",
        "achieved": round(lds_achieved, 1),
        "peak": round(peak["gbs"], 1) if peak else None,
        "unit": "GB/s",
        "frac": round(lds_achieved / peak["gbs"], 5) if peak else None,
        "algorithmic_bytes": lds_bytes,
        "relaxations_per_solve": round(JV_C2_RELAXATIONS / B, 1),
        "peak_probe": peak["probe"] if peak else "probe library not built",
    }
    # The binding resource: each problem is a chain of dependent steps and a
    # launch waits for its slowest problem.  Floor: the slowest problem's
    # sequential search steps, each at least one dependent wave-wide argmin
    # (measured live), against the launch time.
    chain = argmin_chain(device)
    latency = None
    if chain:
        floor_us = JV_C2_CRITICAL_STEPS * chain["cycles_per_round"] / (chain["clock_ghz"] * 1e3)
        latency = {
            "bound": "latency",
            "binding": True,
            "achieved": round(kernel_ms * 1e3, 2),
            "floor": round(floor_us, 2),
            "unit": "us per launch",
            "frac": round(floor_us / (kernel_ms * 1e3), 4),
            "critical_problem_steps": JV_C2_CRITICAL_STEPS,
            "argmin_cycles": round(chain["cycles_per_round"], 1),
            "clock_ghz": round(chain["clock_ghz"], 3),
            "note": "floor = slowest problem's search steps x one dependent wave-wide "
                    "argmin; achieved = the asynchronous entry's launch (fused solve + "
                    "finishing launch)",
        }
    # 16 seeds: problems that fail the certificate replay the reference
    # order, so batches differ in time; each seed's op time is the median of 5
    seeds = {}
    seed_replays = {}
    for seed in range(16):
        c = workloads.jv_uniform(B, N, M, seed=seed).to(device)
        op(c)
        torch.cuda.synchronize()
        seeds[str(seed)] = round(sorted(_events_time_ms(lambda: op(c), 1, stream)
                                        for _ in range(5))[2], 4)
        nrep = ctypes.c_uint32(0)
        lib.tm_jv_dense_batch_f32_sync(c.data_ptr(), B, N, M, outk.data_ptr(), ws.data_ptr(),
                                       ws_bytes, ctypes.byref(nrep), sp)
        seed_replays[str(seed)] = nrep.value
    ordered = sorted(seeds.values())
    seed_stats = {"p50_ms": ordered[len(ordered) // 2],
                  "p90_ms": ordered[int(0.9 * (len(ordered) - 1) + 0.5)],
                  "max_ms": ordered[-1],
                  "min_solves_per_s": round(B / (ordered[-1] * 1e-3), 1),
                  "p50_solves_per_s": round(B / (ordered[len(ordered) // 2] * 1e-3), 1),
                  "replays_per_seed": seed_replays}
    return {
        "solves_per_s": B / (ms_per_step * 1e-3),
        "ms_per_step": ms_per_step,
        "wall_s": wall,
        "kernel_ms": kernel_ms,
        "kernel_solves_per_s": B / (kernel_ms * 1e-3),
        "replays": replays.value,
        "seeds_op_ms": seeds,
        "seed_stats": seed_stats,
        "roofline": {
            "bound": "hbm",
            "binding": False,
            "achieved": round(achieved, 3),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 6),
            "traffic": MEASURED_TRAFFIC["jv_c2"],
            "note": "one read of the input per launch (statistics taken in the solve); "
                    "HBM is not binding, the per-problem dependency chain is "
                    "(latency_roofline); traffic = the fused solve's FETCH/WRITE",
        },
        "lds_roofline": lds_roofline,
        "latency_roofline": latency,
        "cost_sha256": workloads.sha256(cost_cpu),
        "out": out,
    }


def bench_sinkhorn(device, B: int = 16, n_long: int = 200, n_short: int = 20,
                   reps: int = 3) -> dict:
    import workloads

    N = M = 2048
    reg = 0.05
    cost_cpu = workloads.sinkhorn_points(B, N, M, 8, seed=0)
    sha = workloads.sha256(cost_cpu)
    cost = cost_cpu.to(device)
    del cost_cpu
    a = torch.full((B, N), 1.0 / N, device=device)
    b = torch.full((B, M), 1.0 / M, device=device)
    op = torch.ops.transport.log_sinkhorn
    stream = torch.cuda.current_stream(device)
    op(cost, reg, n_short, a, b)
    torch.cuda.synchronize()

    def best(n_iter):
        return min(_events_time_ms(lambda: op(cost, reg, n_iter, a, b), 1, stream)
                   for _ in range(reps))

    t_long = best(n_long)
    t_short = best(n_short)
    per_iter_ms = (t_long - t_short) / (n_long - n_short)
    traffic = {16: MEASURED_TRAFFIC.get("sinkhorn_c4"),
               64: MEASURED_TRAFFIC.get("sinkhorn_b64")}.get(B)
    return {
        "config": {"workload": "log_sinkhorn C4" if B == 16 else "log_sinkhorn C4 shape",
                   "B": B, "N": N, "M": M, "reg": reg, "n_iter": n_long},
        "iters_per_s": 1e3 / per_iter_ms,
        "ms_per_iter": per_iter_ms,
        f"op_ms_{n_long}_iters": t_long,
        "cost_sha256": sha,
        **_sinkhorn_roofline(B, N, M, per_iter_ms, traffic),
    }


def _sinkhorn_roofline(B, N, M, per_iter_ms, traffic) -> dict:
    """One step of this build reads K once (row LSE and the column sums come
    from the same registers): B*N*M*4 algorithmic bytes per iteration."""
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
    }


def bench_jv_c3(device, reps: int = 3) -> dict:
    """C3: (64, 512, 768) squared distances + jitter, 20% +inf (K = 768 kernel)."""
    import workloads

    cost_cpu = workloads.jv_rect_masked()
    cost = cost_cpu.to(device)
    op = torch.ops.assignment.jonker_dense_batch
    op(cost)
    torch.cuda.synchronize()
    ms = _events_time_ms(lambda: op(cost), reps, torch.cuda.current_stream(device)) / reps
    B, N, M = cost.shape
    nbytes = B * N * M * 4 + B * N * 8
    gbs = nbytes / (ms * 1e-3) / 1e9
    res = {"config": {"workload": "jonker_dense_batch C3", "B": B, "N": N, "M": M},
           "solves_per_s": B / (ms * 1e-3), "ms_per_batch": ms,
           "cost_sha256": workloads.sha256(cost_cpu),
           "roofline": {"bound": "hbm", "binding": False, "achieved": round(gbs, 3),
                        "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(gbs / HBM_PEAK_GBS, 6),
                        "traffic": MEASURED_TRAFFIC["jv_c3"],
                        "note": "one wave per problem walks a dependency chain over an "
                                "L2 / Infinity-Cache resident tile; HBM is not binding"}}
    # The binding resource, as for C2: the slowest problem's sequential steps
    # (the reference order the kernel replays), each at least one dependent
    # wave-wide argmin, against the batch time.
    chain = argmin_chain(device)
    if chain:
        floor_ms = JV_C3_CRITICAL_STEPS * chain["cycles_per_round"] / (chain["clock_ghz"] * 1e6)
        res["latency_roofline"] = {
            "bound": "latency", "binding": True, "achieved": round(ms, 3),
            "floor": round(floor_ms, 3), "unit": "ms per batch",
            "frac": round(floor_ms / ms, 4),
            "critical_problem_steps": JV_C3_CRITICAL_STEPS,
            "argmin_cycles": round(chain["cycles_per_round"], 1),
            "clock_ghz": round(chain["clock_ghz"], 3),
            "note": "floor = slowest problem's row-reduction steps + paths + scanned rows "
                    "x one dependent wave-wide argmin; achieved = the op per batch"}
    return res


def bench_jv_c1(device, reps: int = 200) -> dict:
    """C1: (8, 16, 16) U[0,1) through the op, median op time (launch-latency
    bound: eight tiny problems)."""
    import workloads

    cost_cpu = workloads.jv_uniform(8, 16, 16, seed=0)
    cost = cost_cpu.to(device)
    op = torch.ops.assignment.jonker_dense_batch
    for _ in range(5):
        op(cost)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(device)
    ms = sorted(_events_time_ms(lambda: op(cost), 1, stream) for _ in range(reps))[reps // 2]
    return {"config": {"workload": "jonker_dense_batch C1", "B": 8, "N": 16, "M": 16},
            "solves_per_s": 8 / (ms * 1e-3), "ms_per_batch": ms,
            "cost_sha256": workloads.sha256(cost_cpu),
            "note": "median of single op calls; a batch this small is bound by the "
                    "launch and the host wait, not by the solve"}


def bench_jv_compact(device, reps: int = 20) -> dict:
    """jonker_compact_batch on the C2 input (1024, 64, 64), op time per batch."""
    import workloads

    cost = workloads.jv_uniform(1024, 64, 64, seed=0).to(device)
    op = torch.ops.assignment.jonker_compact_batch
    for _ in range(3):
        op(cost)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(device)
    ms = sorted(_events_time_ms(lambda: op(cost), 1, stream) for _ in range(reps))[reps // 2]
    return {"config": {"workload": "jonker_compact_batch on C2", "B": 1024, "N": 64, "M": 64},
            "solves_per_s": 1024 / (ms * 1e-3), "ms_per_batch": ms}


def _c5_inputs():
    import workloads

    N = 16384
    cost = workloads.sinkhorn_points(1, N, N, 8, seed=0)
    a = workloads.dirichlet(1, N, 1.0, seed=1)
    b = workloads.dirichlet(1, N, 1.3, seed=2)
    return cost, a, b


def bench_unbalanced_c5(device, n_long: int = 100, n_short: int = 20) -> dict:
    """C5: unbalanced Sinkhorn on (1, 16384, 16384), reg 0.02, rho 1 (slope)."""
    import workloads

    cost_cpu, a_cpu, b_cpu = _c5_inputs()
    shas = {"cost": workloads.sha256(cost_cpu), "a": workloads.sha256(a_cpu),
            "b": workloads.sha256(b_cpu)}
    N = cost_cpu.shape[1]
    cost, a, b = cost_cpu.to(device), a_cpu.to(device), b_cpu.to(device)
    del cost_cpu
    op = torch.ops.transport.unbalanced_sinkhorn
    stream = torch.cuda.current_stream(device)
    op(cost, 0.02, n_short, 1.0, a, b)
    torch.cuda.synchronize()
    t_long = min(_events_time_ms(lambda: op(cost, 0.02, n_long, 1.0, a, b), 1, stream)
                 for _ in range(2))
    t_short = min(_events_time_ms(lambda: op(cost, 0.02, n_short, 1.0, a, b), 1, stream)
                  for _ in range(2))
    per_iter_ms = (t_long - t_short) / (n_long - n_short)
    res = {"config": {"workload": "unbalanced_sinkhorn C5", "B": 1, "N": N, "M": N,
                      "reg": 0.02, "rho": 1.0},
           "iters_per_s": 1e3 / per_iter_ms, "ms_per_iter": per_iter_ms,
           "input_sha256": shas,
           **_sinkhorn_roofline(1, N, N, per_iter_ms, MEASURED_TRAFFIC.get("sinkhorn_c5"))}
    # the same 1 GiB (the cost) read once by a bare streaming kernel
    ceiling = hbm_read_ceiling(cost)
    if ceiling is not None:
        ceiling["frac_of_ceiling"] = round(res["roofline"]["achieved"] / ceiling["gbs"], 4)
        res["read_ceiling"] = ceiling
    return res


def copy_calibration(device, mib: int = 256, reps: int = 5) -> dict:
    """A plain device copy of known size, for scaling rocprofv3 FETCH/WRITE_SIZE."""
    n = mib * (1 << 20) // 4
    x = torch.rand(n, device=device)
    y = torch.empty_like(x)
    for _ in range(reps):
        y.copy_(x)
    torch.cuda.synchronize()
    return {"copy_bytes_each_way": n * 4, "reps": reps}


def _time_median(fn, budget_s: float, min_runs: int = 5) -> tuple[float, int]:
    fn()  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < min_runs:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_baseline_jv(budget_s: float = 10.0, compact: bool = False, threads: int | None = None,
                    cost=None, label: str = "C2 (1024,64,64) seed 0") -> dict:
    from oracle import jv
    import workloads

    if cost is None:
        cost = workloads.jv_uniform(1024, 64, 64, seed=0).numpy()
    threads = jv.default_threads() if threads is None else threads
    if jv.ref_available():
        fn, kind = (jv.ref_jv_compact_batch if compact else jv.ref_jv_dense_batch), "reference"
    else:
        fn, kind = (jv.jv_compact_batch if compact else jv.jv_dense_batch), "port"
    med, runs = _time_median(lambda: fn(cost, threads), budget_s)
    return {
        "value": cost.shape[0] / med,
        "unit": "solves/s",
        "cores": threads,
        "kind": kind,
        "sample": f"{label}, {runs} runs over ~{budget_s:.0f}s, median",
    }


def cpu_baseline_sinkhorn(n_iter: int = 200) -> dict:
    """C4 on the op-for-op torch restatement: the full 200 iterations once,
    with one iteration timed separately so the fixed cost drops out."""
    from oracle import sinkhorn as sk
    import workloads

    B, N, M = 16, 2048, 2048
    cost = workloads.sinkhorn_points(B, N, M, 8, seed=0)
    a = torch.full((B, N), 1.0 / N)
    t0 = time.perf_counter()
    sk.log_sinkhorn_plan(cost, eps=0.05, n_iter=1, a=a, b=a)
    t1 = time.perf_counter()
    sk.log_sinkhorn_plan(cost, eps=0.05, n_iter=n_iter, a=a, b=a)
    t2 = time.perf_counter()
    per_iter = ((t2 - t1) - (t1 - t0)) / (n_iter - 1)
    return {
        "value": 1.0 / per_iter if per_iter > 0 else None,
        "unit": "iters/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"C4 (16,2048,2048) reg 0.05: {n_iter} iterations once (the full config), "
                  f"slope against 1 iteration; {t2 - t1:.1f} s",
    }


def cpu_baseline_unbalanced_c5(n_iter: int = 20) -> dict:
    """C5 on the op-for-op torch restatement: 20 iterations, slope against 1."""
    from oracle import sinkhorn as sk

    cost, a, b = _c5_inputs()
    t0 = time.perf_counter()
    sk.unbalanced_sinkhorn_plan(cost, eps=0.02, n_iter=1, rho=1.0, a=a, b=b)
    t1 = time.perf_counter()
    sk.unbalanced_sinkhorn_plan(cost, eps=0.02, n_iter=1 + n_iter, rho=1.0, a=a, b=b)
    t2 = time.perf_counter()
    per_iter = ((t2 - t1) - (t1 - t0)) / n_iter
    return {
        "value": 1.0 / per_iter if per_iter > 0 else None,
        "unit": "iters/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"C5 (1,16384,16384) reg 0.02 rho 1: {1 + n_iter} iterations once, "
                  f"slope against 1 iteration; {t2 - t1:.1f} s",
    }


def host_facts() -> dict:
    """CPU model, core counts and versions.  Runs lscpu and hipcc as child
    processes, so main() calls it before anything touches the GPU (a child
    forked from a process with the GPU initialised must not exec)."""
    model = platform.processor() or None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for ln in out.splitlines():
            if ln.startswith("Model name:"):
                model = ln.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    hipcc = None
    try:
        out = subprocess.run(["hipcc", "--version"], capture_output=True, text=True,
                             timeout=30).stdout
        hipcc = next((ln.strip() for ln in out.splitlines() if "HIP version" in ln), None)
    except (OSError, subprocess.SubprocessError):
        pass
    return {
        "cpu_model": model,
        "os_cpu_count": os.cpu_count(),
        "torch_threads": torch.get_num_threads(),
        "torch": torch.__version__,
        "hip": torch.version.hip,
        "hipcc": hipcc,
    }


def _round(d: dict, nd: int) -> dict:
    return {k: (round(v, nd) if isinstance(v, float) else v) for k, v in d.items()}


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
    p.add_argument("--no-host-facts", action="store_true",
                   help="skip the lscpu / hipcc child processes (for runs under a profiler "
                        "that initialises the GPU before the script starts)")
    args = p.parse_args()
    # before the GPU is touched
    host = None if args.copy_calibration or args.no_host_facts else host_facts()
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
    inputs = {"C2": {"generator": "torch.rand U[0,1)", "seed": 0,
                     "sha256": jv_res["cost_sha256"]}}
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
                   "solves_per_s": round(jv_res["kernel_solves_per_s"], 1),
                   "replays": jv_res["replays"]},
        "seeds": {"op_ms": jv_res["seeds_op_ms"], **jv_res["seed_stats"],
                  "note": "op time (median of 5) on seeds 0-15 of the C2 shape; a batch "
                          "with a problem that fails the certificate pays its exact replay"},
        "roofline": jv_res["roofline"],
        "lds_roofline": jv_res["lds_roofline"],
        "latency_roofline": jv_res["latency_roofline"],
    }
    if not args.no_sinkhorn:
        sk = bench_sinkhorn(device)
        inputs["C4"] = {"generator": "sinkhorn_points D=8 / global max, a=b=1/2048",
                        "seed": 0, "sha256": sk.pop("cost_sha256")}
        line["sinkhorn"] = _round(sk, 4)
        # the same kernel shape at B = 64: 1 GiB of K cannot stay in the
        # 256 MB Infinity Cache between iterations
        ctl = bench_sinkhorn(device, B=64, n_long=60, n_short=10)
        ctl.pop("cost_sha256")
        line["sinkhorn_b64_control"] = _round(ctl, 4)
    if not args.no_extra:
        c3 = bench_jv_c3(device)
        inputs["C3"] = {"generator": "jv_rect_masked D=16, 20% +inf", "seed": 0,
                        "sha256": c3.pop("cost_sha256")}
        line["jv_c3"] = _round(c3, 3)
        c5 = bench_unbalanced_c5(device)
        inputs["C5"] = {"generator": "sinkhorn_points D=8; Dirichlet(1) x 1.0 / 1.3",
                        "seeds": {"cost": 0, "a": 1, "b": 2}, "sha256": c5.pop("input_sha256")}
        line["unbalanced_c5"] = _round(c5, 4)
        line["jv_compact_c2"] = _round(bench_jv_compact(device), 4)
        c1 = bench_jv_c1(device)
        inputs["C1"] = {"generator": "torch.rand U[0,1)", "seed": 0,
                        "sha256": c1.pop("cost_sha256")}
        line["jv_c1"] = _round(c1, 5)
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_jv()
        line["cpu_baseline_single_thread"] = cpu_baseline_jv(3.0, threads=1)
        if not args.no_extra:
            import workloads

            line["jv_compact_c2"]["cpu_baseline"] = cpu_baseline_jv(5.0, compact=True)
            line["jv_c1"]["cpu_baseline"] = cpu_baseline_jv(
                2.0, cost=workloads.jv_uniform(8, 16, 16, seed=0).numpy(),
                label="C1 (8,16,16) seed 0")
            line["jv_c3"]["cpu_baseline"] = cpu_baseline_jv(
                5.0, cost=workloads.jv_rect_masked().numpy(),
                label="C3 (64,512,768) 20% +inf seed 0")
            line["unbalanced_c5"]["cpu_baseline"] = cpu_baseline_unbalanced_c5()
        if not args.no_sinkhorn:
            line["sinkhorn"]["cpu_baseline"] = cpu_baseline_sinkhorn()
    host = host or {}
    host["gpu"] = torch.cuda.get_device_name(0)
    line["host"] = host
    line["inputs"] = inputs
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
