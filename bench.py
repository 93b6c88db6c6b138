#!/usr/bin/env python3
"""Throughput of the MI355X Chambolle--Pock projection on one GPU.

Workload (the headline configuration, "config2"): n = 4096 variables, 1024
equality + 2048 inequality rows of 8 random columns each, box bounds [-1, 1]
as 8192 singleton rows (presolved), batch 1024, float64, accelerated CP,
2000 fixed iterations.  One step = one ``purin_cp_project`` call on the whole
batch (bound presolve, 2000 CP iterations, final diagnostics, dual recovery,
statuses), with the inputs already resident in device memory.

Printed: one JSON line with the driver's fields plus
  roofline      the dominant kernel (the resident CP kernel; the column pass when
                the streaming passes run) against HBM peak: its algorithmic bytes
                per launch over its average duration, measured with HIP events
                on the launch stream (instrumented replay), and its HBM traffic
                from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary;
  cpu_baseline  the NumPy oracle on a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(w, samples, iterations):
    """NumPy oracle on the first ``samples`` samples for ``iterations`` CP iterations."""
    from oracle import projection as op

    canon = op.Canonical(n=w.n, me=w.me, rows=w.rows(), coef=w.coefs())
    target = np.asarray(w.target[:samples], np.float64)
    rhs = np.tile(w.rhs, (samples, 1))
    cfg = op.Config(accelerated=w.accelerated, max_iterations=iterations, early_stop=False)
    t0 = time.perf_counter()
    op.solve(canon, target, rhs, cfg)
    dt = time.perf_counter() - t0
    # projections/s at the full iteration count: the loop dominates and scales linearly
    per_projection = dt / samples * (w.iterations / iterations)
    return {
        "value": 1.0 / per_projection,
        "unit": "projections/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"NumPy/scipy oracle (oracle/projection.py), first {samples} samples x "
                   f"{iterations} of {w.iterations} iterations, scaled linearly to "
                   f"{w.iterations}; {dt:.1f} s on {_cpu_model()} "
                   f"(affinity {len(os.sched_getaffinity(0))} cores, 1 used)"),
    }


def traffic_from_profiles(kernel, batch, iterations):
    """HBM bytes per dispatch of ``kernel`` from the committed rocprofv3 PMC summary
    (FETCH_SIZE and WRITE_SIZE runs, calibrated against a plain copy), or None when
    the summary is absent or was taken on another workload size."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        "traffic_config2.json")
    try:
        with open(path) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return None
    wl = data.get("workload", {})
    if wl.get("batch") != batch or wl.get("iterations") != iterations:
        return None
    return data.get("hbm_bytes_per_dispatch", {}).get(kernel)


def copy_calibration(torch, mib):
    """A plain copy of known size: its counter readings per dispatch, divided by
    ``mib`` MiB read and written, are the scale factors for FETCH_SIZE / WRITE_SIZE."""
    n = mib * (1 << 20) // 8
    src = torch.ones(n, dtype=torch.float64, device="cuda:0")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n * 8, "dispatches": 3}), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--batch", type=int, default=1024)
    ap.add_argument("--iterations", type=int, default=2000)
    ap.add_argument("--cpu-samples", type=int, default=64)
    ap.add_argument("--cpu-iterations", type=int, default=500)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-streaming", action="store_true",
                    help="skip the streaming two-pass comparison run")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="only run a plain device-to-device copy of this many MiB (3 times); "
                         "its FETCH_SIZE / WRITE_SIZE counters calibrate the traffic figures")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: the batch shards across GPUs "
                          "with no per-iteration communication, so run --gpus 1 per GPU"}))
        sys.exit(2)

    import torch

    if args.copy_calibration_mib:
        copy_calibration(torch, args.copy_calibration_mib)
        return

    from purin_amd import workloads
    from purin_amd.plan import Plan

    w = workloads.config2(args.batch)
    w.iterations = args.iterations
    B, n = w.target.shape
    plan = Plan(w.n, w.me, w.rows_total - w.me, w.indptr, w.indices, w.data,
                dtype=torch.float64, accelerated=True, device="cuda:0")
    m = plan.m
    dev = torch.device("cuda:0")
    target = torch.as_tensor(w.target, device=dev)
    rhs = torch.as_tensor(np.tile(w.rhs, (B, 1)), device=dev)
    kw = dict(max_iterations=args.iterations, early_stop=False, shared_bounds=True)

    for _ in range(args.warmup):
        plan.project(target, rhs, **kw)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(args.steps):
        out = plan.project(target, rhs, **kw)
    e1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = e0.elapsed_time(e1) / args.steps
    value = B / (ms_per_step / 1e3)
    status = out.status.cpu().numpy()

    # instrumented replay: HIP events around the iteration kernels' launches
    plan.project(target, rhs, timing=True, **kw)
    torch.cuda.synchronize()
    tm = plan.last_timing()
    iters = max(int(tm["iterations"]), 1)
    ws = 8
    bytes_row = B * ws * (n + 3 * m)        # gather ybar (n), read d, r (2m), write d (m)
    bytes_col = B * ws * (4 * n + m)        # gather d+ (m), read y, yhat (2n), write y, ybar (2n)
    bytes_iter = B * ws * (5 * n + 3 * m)   # the per-iteration contract figure
    iter_ms = tm["loop_ms"] / iters
    if tm["resident"]:
        # one launch runs every iteration with the state on chip
        dominant, dom_bytes, dom_ms = "k_resident", bytes_iter * iters, tm["loop_ms"]
        row_ms = col_ms = None
    else:
        row_ms, col_ms = tm["row_ms"] / iters, tm["col_ms"] / iters
        dominant = "k_col_pass" if col_ms >= row_ms else "k_row_pass"
        dom_bytes, dom_ms = (bytes_col, col_ms) if dominant == "k_col_pass" else (bytes_row, row_ms)
    achieved = dom_bytes / (dom_ms / 1e3) / 1e9
    traffic = traffic_from_profiles(dominant, B, args.iterations)
    # the streaming two-pass path on the same inputs, for comparison
    streaming_ms = None
    if not args.no_streaming:
        e2 = torch.cuda.Event(enable_timing=True)
        e3 = torch.cuda.Event(enable_timing=True)
        e2.record(stream)
        plan.project(target, rhs, streaming=True, **kw)
        e3.record(stream)
        torch.cuda.synchronize()
        streaming_ms = e2.elapsed_time(e3)
    line = {
        "metric": "CP projections/sec (n=4096, batch 1024, fp64) + achieved HBM GB/s % of peak",
        "value": value,
        "unit": "projections/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64",
        "data": "synthetic (config2 generator, numpy default_rng seed 2)",
        "config": {
            "workload": "config2: n=4096, 1024 eq + 2048 ineq rows x 8 cols, 8192 bound rows, "
                        "batch 1024, fp64, accelerated CP, fixed iterations, full projection",
            "n": n, "kept_rows": m, "bound_rows": int(plan.info.bound_rows),
            "nnz_kept": int(plan.info.nnz_kept), "batch": B, "iterations": args.iterations,
            "parallelism": "1 GPU (batch-parallel)",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": dominant,
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic,
            "bytes_per_launch": dom_bytes,
            "avg_launch_ms": dom_ms,
        },
        "iteration": {
            "cp_iterations_per_s": args.iterations * 1e3 / ms_per_step,
            "resident_kernel": bool(tm["resident"]),
            "streaming_passes_ms_per_step": streaming_ms,
            "row_pass_ms": row_ms,
            "col_pass_ms": col_ms,
            "iteration_ms": iter_ms,
            "algorithmic_bytes": bytes_iter,
            "achieved_GBs": bytes_iter / (iter_ms / 1e3) / 1e9,
            "frac_of_hbm_peak": bytes_iter / (iter_ms / 1e3) / 1e9 / HBM_PEAK_GBS,
        },
        "statuses": {str(k): int(v) for k, v in zip(*np.unique(status, return_counts=True))},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(w, args.cpu_samples, args.cpu_iterations)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
