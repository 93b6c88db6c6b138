#!/usr/bin/env python3
"""Throughput of the MI355X Chambolle--Pock projection on one GPU.

Default workload (the headline configuration, "config2"): n = 4096 variables,
1024 equality + 2048 inequality rows of 8 random columns each, box bounds
[-1, 1] as 8192 singleton rows (presolved), batch 1024, float64, accelerated
CP, 2000 fixed iterations.  One step = one ``purin_cp_project`` call on the
whole batch (bound presolve, 2000 CP iterations, final diagnostics, dual
recovery, statuses), with the inputs already resident in device memory.
``--config 3`` / ``--config 4`` measure the network-flow WeightedDistance
(fp64, B=256, 3000 iterations) and high-batch fp32 (B=65536, 500 iterations)
configurations the same way.

Printed: one JSON line with the driver's fields plus
  roofline      the dominant kernel against the resource that bounds it.  The
                resident CP kernel keeps the iterate on chip, so HBM does not
                bound it: its bound is the L2 -> CU stream of the shared matrix
                (chunk-stream bytes per launch over the launch's duration, HIP
                events on the launch stream) against the best rate the
                ``k_probe_stream`` ceiling probe (libpurin_probe.so) reaches at
                the same launch shape, measured in the same run; ``lds`` gives
                its LDS bytes against the ``k_probe_lds`` ceiling, and ``hbm``
                the algorithmic state bytes against the 8 TB/s HBM peak (context
                only).  For the streaming passes (config 3) the bound is HBM.
                ``traffic`` is the HBM bytes per launch from the committed
                rocprofv3 FETCH_SIZE / WRITE_SIZE summary;
  per_sample_bounds  the same projection with per-sample bounds (the kernels a
                caller whose bound rows depend on the parameters runs);
  purin_api     the same projection through the PURIN-API front end
                (``Distance(problem).prepare(batch_size=...)``), which picks the
                shared-bounds kernels itself for constant bound rows;
  adjoint       (config2) the implicit VJP w.r.t. the candidates and b, h
                (``purin_cp_adjoint``, cotangents N(0,1) from seed 5) at the
                2000-iteration state with eligibility forced on, timed separately
                from the forward;
  cpu_baseline  the checker's C restatement of the CP loop (bit-equal to the NumPy
                oracle) on a bounded sample of the same workload, on the threads
                this process may use (``value``) and one core (``one_core``);
  cpu_baseline_adjoint  the NumPy oracle's GMRES pullback (the checker) on a
                bounded sample of the config5 VJP, one thread.
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
PROBE_LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "purin_amd",
                         "libpurin_probe.so")

METRICS = {
    2: "CP projections/sec (n=4096, batch 1024, fp64) + achieved HBM GB/s % of peak",
    3: "CP projections/sec (network flow n=40000 edges, 10000 nodes, batch 256, fp64, "
       "WeightedDistance) + achieved HBM GB/s % of peak",
    4: "CP projections/sec (n=1024, batch 65536, fp32) + achieved HBM GB/s % of peak",
}


# CPU-baseline samples (one core, all threads) for the headline configuration
# and, smaller, for the configurations timed beside config2 in the default line
CPU_SAMPLES = {2: (64, 512), 3: (4, 64), 4: (256, 4096)}
CPU_SAMPLES_OTHER = {3: (2, 16), 4: (64, 1024)}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def weighted_values(w):
    """CSR values with the metric change of variables (coefficients times 1/sqrt(D_j))."""
    if w.metric is None:
        return w.data, None
    root = np.sqrt(np.asarray(w.metric, np.float64))
    return w.data / root[w.indices], root


def cpu_baseline(w, samples_one, samples_all):
    """The C restatement of the CP loop (oracle/cp_loop.c, bit-equal to the NumPy
    oracle) at the full iteration count: ``samples_one`` samples on one core, then
    ``samples_all`` samples on every core this process may use (at most 16)."""
    from oracle import cloop
    from oracle import projection as op

    values, root = weighted_values(w)
    rows = [list(w.indices[w.indptr[i]:w.indptr[i + 1]]) for i in range(w.rows_total)]
    coef = [list(values[w.indptr[i]:w.indptr[i + 1]]) for i in range(w.rows_total)]
    canon = op.Canonical(n=w.n, me=w.me, rows=rows, coef=coef)
    cfg = op.Config(accelerated=w.accelerated, max_iterations=w.iterations, early_stop=False)
    affinity = len(os.sched_getaffinity(0))
    cores = cpu_threads()

    def leg(samples, threads):
        target = np.asarray(w.target[:samples], w.dtype)
        if root is not None:
            target = target * root.astype(w.dtype)
        rhs = np.tile(w.rhs, (samples, 1)).astype(w.dtype)
        prep = cloop.prepare(canon, target, rhs, cfg, w.dtype)
        _, _, seconds = cloop.run(prep, w.iterations, w.accelerated, threads=threads)
        return samples / seconds, seconds

    one, t_one = leg(samples_one, 1)
    full, t_full = leg(samples_all, cores)
    return {
        "value": full,
        "unit": "projections/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"C restatement of the CP loop (oracle/cp_loop.c, OpenMP over samples; "
                   f"set-up by the NumPy oracle, untimed), {w.iterations} iterations: "
                   f"{samples_all} samples on {cores} threads (every core of this "
                   f"process's CPU set: {affinity} in the affinity mask"
                   + (f", OMP_NUM_THREADS={os.environ['OMP_NUM_THREADS']}"
                      if os.environ.get("OMP_NUM_THREADS") else "")
                   + f") in {t_full:.1f} s; {samples_one} samples on 1 thread in {t_one:.1f} s "
                   f"= {one:.2f} projections/s; {_cpu_model()}"),
        "one_core": one,
        "affinity_cores": affinity,
    }


def cpu_threads():
    """Threads for the all-core CPU leg: every core in this process's affinity
    mask, or fewer when OMP_NUM_THREADS caps the process (the GPU box sets it to
    the box's CPU share)."""
    cores = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        cores = min(cores, int(env))
    return max(1, cores)


def cpu_baseline_adjoint(w, plan, out_y, out_dual, lower, upper, rhs_k, samples):
    """The NumPy oracle's implicit VJP (bounds.py:80-165 with the CGS2 GMRES of
    operators.py:792-1125; the checker of the GPU adjoint) on ``samples`` samples
    of the config5 workload, linearised at the same forward state, one thread."""
    from threadpoolctl import threadpool_limits

    from oracle import adjoint as oadj
    from oracle import projection as op

    cfg = op.Config(accelerated=True, max_iterations=w.iterations, early_stop=False)
    one = op.Canonical(n=w.n, me=w.me, rows=w.rows(), coef=w.coefs())
    pre = op.presolve(one, w.rhs[None, :], cfg, np.float64)
    ksup, kmask = pre.support[pre.rows], pre.mask[pre.rows]
    sub = np.arange(samples)
    args = (pre.kept_values[0], ksup, kmask, w.me, out_y[sub], out_dual[sub],
            np.ones(samples, bool), w.target[sub], rhs_k[sub],
            np.broadcast_to(lower, (samples, w.n)), np.broadcast_to(upper, (samples, w.n)),
            w.cotangent[sub], cfg)
    with threadpool_limits(limits=1):
        t0 = time.perf_counter()
        res = oadj.adjoint(*args)
        seconds = time.perf_counter() - t0
    info = np.asarray(res.info)
    return {
        "value": samples / seconds,
        "unit": "VJPs/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"NumPy oracle adjoint (oracle/adjoint.py: mask-form pullback, batched CGS2 "
                   f"GMRES restart 30, max 100, tol 1e-9) on {samples} samples of the config5 "
                   f"VJP at the {w.iterations}-iteration state, eligibility forced, one thread, "
                   f"in {seconds:.1f} s (GMRES info {dict(zip(*np.unique(info, return_counts=True)))}); "
                   f"{_cpu_model()}"),
    }


def traffic_from_profiles(config, kernel, batch, iterations):
    """HBM bytes per dispatch of ``kernel`` from the committed rocprofv3 PMC summary
    (FETCH_SIZE and WRITE_SIZE runs, calibrated against a plain copy), or None when
    the summary is absent or was taken on another workload size."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        f"traffic_config{config}.json")
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


def probe_ceilings(torch, groups, lds_bytes, stream_bytes_iter):
    """Best rates (GB/s) of the ceiling probes (libpurin_probe.so) at the resident
    kernel's launch shape: ``groups`` workgroups of 1024 threads.  The L2 -> CU
    chunk stream is probed with the kernel's per-wavefront stream length and its
    dynamic LDS (one workgroup per CU) and with 64 KiB (two per CU), 1, 2 and 4
    chunks in flight; LDS reads with 1 to 8 conflict-free ds_read_b128 in flight.
    Each variant: one warm-up launch, then the mean of 3 timed launches (HIP
    events on the current stream)."""
    import ctypes as C

    lib = C.CDLL(PROBE_LIB)
    vp, i64, i32 = C.c_void_p, C.c_int64, C.c_int32
    lib.purin_probe_stream.argtypes = [vp, vp, i64, i64, i32, i32, i32, i32, i32, vp, i64,
                                       C.POINTER(C.c_double)]
    lib.purin_probe_lds.argtypes = [vp, i32, i32, i32, i32, i32, vp, i64, C.POINTER(C.c_double)]
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    dev = torch.device("cuda:0")
    sink = torch.zeros(1024, dtype=torch.int32, device=dev)
    chunk = 3072
    wave_chunks = max(4, int(round(stream_bytes_iter / 16 / chunk / 4)) * 4)
    buf = torch.zeros(16 * wave_chunks * chunk, dtype=torch.uint8, device=dev)
    per_iter = groups * 16 * wave_chunks * chunk
    iters = max(1, int(300e9 // per_iter))
    ms = C.c_double()
    l2 = []
    for lds in sorted({int(lds_bytes), 65536}):
        for unroll in (1, 2, 4):
            for reps in (1, 3):
                rc = lib.purin_probe_stream(stream, C.c_void_p(buf.data_ptr()), buf.numel(),
                                            wave_chunks, iters, groups, lds, unroll, reps,
                                            C.c_void_p(sink.data_ptr()), sink.numel() * 4,
                                            C.byref(ms))
                if rc != 0:
                    raise RuntimeError(f"purin_probe_stream failed ({rc})")
            l2.append({"lds_bytes": lds, "unroll": unroll, "ms": ms.value,
                       "GBs": per_iter * iters / (ms.value / 1e3) / 1e9})
    lds_rates = []
    lds_iter = groups * 1024 * 16
    for lds in sorted({max(int(lds_bytes), 65536), 65536}):
        for unroll in (1, 2, 4, 8):
            it = max(1, int(600e9 // (lds_iter * unroll)))
            for reps in (1, 3):
                rc = lib.purin_probe_lds(stream, it, groups, lds, unroll, reps,
                                         C.c_void_p(sink.data_ptr()), sink.numel() * 4,
                                         C.byref(ms))
                if rc != 0:
                    raise RuntimeError(f"purin_probe_lds failed ({rc})")
            lds_rates.append({"lds_bytes": lds, "unroll": unroll, "ms": ms.value,
                              "GBs": lds_iter * unroll * it / (ms.value / 1e3) / 1e9})
    best_l2 = max(l2, key=lambda r: r["GBs"])
    best_lds = max(lds_rates, key=lambda r: r["GBs"])
    return {"l2": best_l2, "lds": best_lds, "l2_all": l2, "lds_all": lds_rates,
            "wave_chunks": wave_chunks, "groups": groups}


def adjoint_bytes(batch, ws, width, steps, restart):
    """Algorithmic bytes of the batched GMRES: B*ws*(k+2)*W for Arnoldi step k of a
    cycle (read v_k and the k-vector prefix once, write the new vector) plus
    B*ws*38*W per cycle for its set-up and finish."""
    total, done = 0, 0
    while done < steps:
        length = min(restart, steps - done)
        total += sum(k + 2 for k in range(1, length + 1)) + 38
        done += length
    return batch * ws * width * total


def adjoint_streamed_bytes(batch, ws, n, m, steps, restart):
    """Bytes the adjoint's kernels stream by construction, in vectors of W = 2n + m
    rows of B samples.  Per Arnoldi step with a k-vector prefix: the dot pass
    reads the prefix and the image (k + 1), the update-and-dot pass reads them
    again and writes the next raw vector (k + 2), and the operator moves about 4.
    Per cycle: the correction reads the prefix once, and the residual,
    acceptance and norms move about 40."""
    W = 2 * n + m
    total, done = 0, 0
    while done < steps:
        length = min(restart, steps - done)
        total += sum(2 * k + 3 + 4 for k in range(1, length + 1)) + length + 40
        done += length
    return batch * ws * W * total


MODES = {
    "values": "CP projections/sec with per-sample coefficients (config2 rows, values (B, nnz) "
              "per sample, batch 1024, fp64) + achieved HBM GB/s % of peak",
    "qp": "diagonal-QP solves/sec (config2 general rows, box [-1,1], per-sample q, c, batch "
          "1024, fp64) + achieved HBM GB/s % of peak",
    "dense": "dense-adapter solves/sec (n=256, 32 eq + 96 ineq dense rows per sample, batch "
             "4096, fp64) + achieved HBM GB/s % of peak",
}


def run_mode(args, torch):
    """The widened paths on config2-sized data: per-sample coefficients
    (purin_cp_project_values), the general diagonal QP (purin_cp_qp_solve) and the
    dense adapter (purin_cp_dense_solve).  Streaming passes; the roofline is the
    dominant pass with its algorithmic bytes, which include the per-sample
    coefficients each pass reads (B * ws * nnz) where the coefficients are per
    sample (values, dense); the QP here uses the plan's shared coefficients."""
    from purin_amd import workloads
    from purin_amd.plan import Plan

    dev = torch.device("cuda:0")
    rng = np.random.default_rng(7)
    ws = 8
    if args.mode in ("values", "qp"):
        w = workloads.config2(args.batch or 1024)
        iters = args.iterations or w.iterations
        B = w.target.shape[0]
        if args.mode == "values":
            plan = Plan(w.n, w.me, w.rows_total - w.me, w.indptr, w.indices, w.data,
                        dtype=torch.float64, accelerated=True, device="cuda:0")
            scale = 1.0 + 0.1 * rng.uniform(-1.0, 1.0, (B, w.indptr[-1]))
            values = torch.as_tensor(w.data[None, :] * scale, device=dev)
            target = torch.as_tensor(w.target, device=dev)
            rhs = torch.as_tensor(np.tile(w.rhs, (B, 1)), device=dev)
            call = lambda timing=False, streaming=False, early=False: plan.project(
                target, rhs, values=values, timing=timing, streaming=streaming,
                max_iterations=iters, early_stop=early, tolerance=1e-9)
            extra_n = 0
        else:
            general = w.me + int(w.info["mi_general"])
            indptr = w.indptr[:general + 1]
            nnz = int(indptr[-1])
            plan = Plan(w.n, w.me, general - w.me, indptr, w.indices[:nnz], w.data[:nnz],
                        dtype=torch.float64, accelerated=True, bound_presolve=False,
                        device="cuda:0")
            q = torch.as_tensor(rng.uniform(0.5, 2.0, (B, w.n)), device=dev)
            c = -q * torch.as_tensor(w.target, device=dev)
            rhs = torch.as_tensor(np.tile(w.rhs[:general], (B, 1)), device=dev)
            lo = torch.full((B, w.n), -1.0, dtype=torch.float64, device=dev)
            hi = torch.full((B, w.n), 1.0, dtype=torch.float64, device=dev)
            call = lambda timing=False, streaming=False, early=False: plan.qp_solve(
                q, c, rhs, lo, hi, max_iterations=iters, early_stop=early, tolerance=1e-9,
                timing=timing, streaming=streaming)
            extra_n = 1  # q and c replace the candidates: one more n-vector per iteration
        n, m, nnz = w.n, plan.m, int(plan.info.nnz_kept)
        # the QP with the plan's own coefficients reads one shared copy of them
        coef_nnz = 0 if args.mode == "qp" else nnz
        workload = {"values": "config2 rows and sparsity, per-sample values = shared values x "
                              "(1 + 0.1 U(-1,1)) (seed 7), batch 1024, fp64, accelerated CP, "
                              f"{iters} fixed iterations, full projection",
                    "qp": "config2's 3072 general rows (the plan's shared coefficients), "
                          "box [-1,1], q ~ U(0.5,2), c = -q yhat (seed 7), batch 1024, fp64, "
                          f"accelerated CP, {iters} fixed iterations"}[args.mode]
    else:
        B = args.batch or 4096
        n, me, mi = 256, 32, 96
        iters = args.iterations or 500
        A = rng.normal(size=(B, me, n))
        C = rng.normal(size=(B, mi, n))
        x0 = rng.uniform(-0.3, 0.3, (B, n))
        b = np.einsum("bmn,bn->bm", A, x0)
        d = np.einsum("bmn,bn->bm", C, x0) + rng.uniform(0.1, 1.0, (B, mi))
        rows = [list(range(n))] * (me + mi)
        indptr = np.zeros(me + mi + 1, np.int64)
        indptr[1:] = np.cumsum([n] * (me + mi))
        plan = Plan(n, me, mi, indptr, np.tile(np.arange(n, dtype=np.int32), me + mi),
                    np.ones(indptr[-1]), dtype=torch.float64, bound_presolve=False,
                    row_scaling=False, norm_bound=False, device="cuda:0")
        values = torch.as_tensor(np.concatenate((A, C), axis=1).reshape(B, -1), device=dev)
        q = torch.as_tensor(rng.uniform(0.5, 2.0, (B, n)), device=dev)
        c = torch.as_tensor(rng.normal(size=(B, n)), device=dev)
        rhs = torch.as_tensor(np.concatenate((b, d), axis=1), device=dev)
        lo = torch.full((B, n), -1.0, dtype=torch.float64, device=dev)
        hi = torch.full((B, n), 1.0, dtype=torch.float64, device=dev)
        call = lambda timing=False: plan.dense_solve(q, c, rhs, lo, hi, values=values,
                                                     max_iterations=iters, early_stop=False,
                                                     timing=timing)
        m, nnz, extra_n = me + mi, int(indptr[-1]), 1
        coef_nnz = nnz
        workload = (f"dense adapter: n={n}, {me} eq + {mi} ineq dense rows per sample N(0,1), "
                    f"feasible rhs, box [-1,1], q ~ U(0.5,2), c ~ N(0,1) (seed 7), batch {B}, "
                    f"fp64, fixed-step CP, {iters} fixed iterations")
    for _ in range(args.warmup):
        call()
    ms_per_step, _ = time_calls(torch, call, args.steps)
    call(True)
    torch.cuda.synchronize()
    tm = plan.last_timing()
    it = max(int(tm["iterations"]), 1)
    if tm["resident"]:  # the diagonal QP's fixed iterations on the resident kernel
        resident_mode_line(args, torch, plan, call, tm, B, n, m, nnz, ws, iters, ms_per_step,
                         workload)
        return
    row_ms, col_ms = tm["row_ms"] / it, tm["col_ms"] / it
    # these entry points take per-sample bounds: the column pass reads lower and upper (2n)
    bytes_row = B * ws * (n + 3 * m + coef_nnz)               # gather ybar, d, r, d+, per-sample entries
    bytes_col = B * ws * ((6 + extra_n) * n + m + coef_nnz)   # y, yhat (or q, c), bounds, writes, d+, entries
    if tm["linear_kybar"]:
        # K ybar formed from K y: the row pass reads and writes K y (2m), the column
        # pass writes no ybar (n)
        bytes_row += B * ws * 2 * m
        bytes_col -= B * ws * n
    col_kernel = "k_col_pass_q" if tm["narrow_columns"] else "k_col_pass"
    dominant = col_kernel if col_ms >= row_ms else "k_row_pass"
    dom_bytes, dom_ms = (bytes_col, col_ms) if dominant == col_kernel else (bytes_row, row_ms)
    achieved = dom_bytes / (dom_ms / 1e3) / 1e9
    bytes_iter = B * ws * ((7 + extra_n) * n + 3 * m + 2 * coef_nnz)
    iter_ms = tm["loop_ms"] / it
    line = {
        "metric": MODES[args.mode], "value": B / (ms_per_step / 1e3),
        "unit": "solves/s" if args.mode != "values" else "projections/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f64",
        "data": "synthetic (numpy default_rng)",
        "config": {"workload": workload, "n": n, "rows": m, "nnz": nnz, "batch": B,
                   "iterations": iters, "parallelism": "1 GPU (batch-parallel)"},
        "roofline": {"bound": "hbm", "kernel": dominant, "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": None, "bytes_per_launch": dom_bytes, "avg_launch_ms": dom_ms},
        "iteration": {"row_pass_ms": row_ms, "col_pass_ms": col_ms, "iteration_ms": iter_ms,
                      "algorithmic_bytes": bytes_iter,
                      "achieved_GBs": bytes_iter / (iter_ms / 1e3) / 1e9,
                      "frac_of_hbm_peak": bytes_iter / (iter_ms / 1e3) / 1e9 / HBM_PEAK_GBS},
    }
    print(json.dumps(line), flush=True)


def resident_mode_line(args, torch, plan, call, tm, B, n, m, nnz, ws, iters, ms_per_step,
                       workload):
    """The ``--mode qp`` / ``--mode values`` line when the fixed iterations run on
    the resident kernel.  The diagonal QP (the plan's shared coefficients) is
    priced, like the headline, on the L2 -> CU matrix stream against the
    same-run stream probe; per-sample coefficients on the HBM bytes of the
    tiles' coefficient streams (each tile reads its samples' coefficients once
    per iteration, in the plan's stream order) against the HBM peak.  The
    state bytes on HBM terms are context; the streaming passes on the same
    inputs are timed beside it."""
    info = plan.info
    bt = int(info.resident_tile_samples)
    pad = 64 * (2 if ws == 8 else 4)
    tiles = -(-B // pad) * pad // bt
    sbytes = int(info.resident_stream_bytes)
    chunk = 64 * 16 + 64 * 4 * ws
    loop_ms = tm["loop_ms"]
    streaming_ms, _ = time_calls(torch, lambda: call(streaming=True), 1)
    if args.mode == "qp":
        l2_bytes = tiles * iters * sbytes
        ceil = probe_ceilings(torch, tiles, (n + 1 + m + 1) * 16, sbytes)
        l2_rate = l2_bytes / (loop_ms / 1e3) / 1e9
        # q, c (2n) replace the candidates: B ws ((7 + 1) n + 3 m) per iteration
        bytes_iter = B * ws * (8 * n + 3 * m)
        roofline = {"bound": "l2", "kernel": "k_resident (diagonal QP)", "achieved": l2_rate,
                    "peak": ceil["l2"]["GBs"], "unit": "GB/s",
                    "frac": l2_rate / ceil["l2"]["GBs"], "traffic": None,
                    "bytes_per_launch": l2_bytes, "avg_launch_ms": loop_ms,
                    "what": f"L2 -> CU bytes of the shared matrix's chunk streams: {sbytes} B "
                            f"per workgroup per iteration x {tiles} workgroups x {iters} "
                            "iterations",
                    "peak_source": "measured in this run: best rate of the k_probe_stream "
                                   f"ceiling probe at {tiles} workgroups of 1024 threads"}
    else:
        # every tile reads its coefficient stream once per iteration: 4 entries per
        # lane per chunk, bt samples each
        cbytes = tiles * iters * (sbytes // chunk) * 256 * bt * ws
        rate = cbytes / (loop_ms / 1e3) / 1e9
        bytes_iter = B * ws * (7 * n + 3 * m + 2 * nnz)
        roofline = {"bound": "hbm", "kernel": "k_resident (per-sample coefficients)",
                    "achieved": rate, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": rate / HBM_PEAK_GBS, "traffic": None, "bytes_per_launch": cbytes,
                    "avg_launch_ms": loop_ms,
                    "what": f"HBM bytes of the tiles' coefficient streams: {sbytes // chunk} "
                            f"chunks x 256 entries x {bt} samples x {ws} B per workgroup per "
                            f"iteration x {tiles} workgroups x {iters} iterations (the "
                            "iterate stays on chip)"}
    roofline["hbm_context"] = {
        "achieved": bytes_iter * iters / (loop_ms / 1e3) / 1e9, "peak": HBM_PEAK_GBS,
        "bytes_per_launch": bytes_iter * iters,
        "note": "algorithmic bytes of the streaming formulation per iteration (state "
                "vectors" + (" and per-sample coefficients" if args.mode == "values" else "")
                + "); the state stays on chip (context only)"}
    line = {
        "metric": MODES[args.mode], "value": B / (ms_per_step / 1e3),
        "unit": "solves/s" if args.mode == "qp" else "projections/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f64",
        "data": "synthetic (numpy default_rng)",
        "config": {"workload": workload, "n": n, "rows": m, "nnz": nnz, "batch": B,
                   "iterations": iters, "parallelism": "1 GPU (batch-parallel)"},
        "roofline": roofline,
        "iteration": {"resident_kernel": True, "iteration_ms": loop_ms / iters,
                      "streaming_passes_ms_per_step": streaming_ms,
                      "streaming_passes_value": B / (streaming_ms / 1e3)},
    }
    # the default loop (early stop at tolerance 1e-9, freezing,
    # stationarity) on the same inputs, resident and streaming
    call(early=True)
    early_ms, res = time_calls(torch, lambda: call(early=True, timing=True), 1)
    early_resident = plan.last_timing()["resident"]
    early_iters = int(res.iterations.max().item())
    early_streaming_ms, _ = time_calls(torch, lambda: call(early=True, streaming=True), 1)
    line["early_stop"] = {
        "what": "the same solve with early stop at tolerance 1e-9 (the stop test every "
                "iteration, freezing, stationarity)",
        "ms_per_step": early_ms, "value": B / (early_ms / 1e3),
        "resident_kernel": bool(early_resident), "iterations_max": early_iters,
        "streaming_passes_ms_per_step": early_streaming_ms,
        "streaming_passes_value": B / (early_streaming_ms / 1e3)}
    print(json.dumps(line), flush=True)


def purin_api_timing(torch, w, values, root, target, steps):
    """One projection through the PURIN-API front end (``Distance`` /
    ``WeightedDistance`` over a ``MatrixProblem`` of the workload's rows), timed
    per call with the inputs on the device."""
    import scipy.sparse as sp

    from purin_amd.config import ChambollePockConfig
    from purin_amd.problems import MatrixProblem
    from purin_amd.projection import Distance, WeightedDistance

    me, M = w.me, w.rows_total
    A = sp.csr_matrix((w.data, w.indices, w.indptr), shape=(M, w.n))
    problem = MatrixProblem(P=sp.identity(w.n, format="csr"), q0=np.zeros(w.n), A_eq=A[:me],
                            b_eq0=w.rhs[:me], A_ineq=A[me:], b_ineq0=w.rhs[me:])
    cfg = ChambollePockConfig(accelerated=w.accelerated, max_iterations=w.iterations,
                              early_stop=False)
    B = w.target.shape[0]
    tdtype = torch.float64 if w.dtype == np.float64 else torch.float32
    if w.metric is not None:
        layer = WeightedDistance(problem, tuple(np.asarray(w.metric, np.float64)),
                                 config=cfg).prepare(batch_size=B, dtype=tdtype)
    else:
        layer = Distance(problem, config=cfg).prepare(batch_size=B, dtype=tdtype)
    y_hat = torch.as_tensor(w.target, device="cuda:0")
    with torch.no_grad():
        layer(y_hat)
        ms, _ = time_calls(torch, lambda: layer(y_hat), steps)
    return {"ms_per_step": ms, "value": B / (ms / 1e3), "unit": "projections/s",
            "shared_bounds": layer.shared_bounds,
            "what": "Distance(MatrixProblem(rows), ChambollePockConfig(accelerated, "
                    "max_iterations, early_stop=False)).prepare(batch_size=B)(y_hat)"}


def time_calls(torch, fn, count):
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(count):
        out = fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / count, out


def measure(args, torch, config, *, steps, warmup, headline):
    """Time ``purin_cp_project`` on one configuration; returns (line, context).

    ``headline``: the configuration of the driver's line (the command-line
    batch / iteration overrides apply, and the extra legs run)."""
    from purin_amd import workloads
    from purin_amd.plan import Plan

    make = {2: workloads.config2, 3: workloads.config3, 4: workloads.config4}[config]
    w = make(args.batch) if (args.batch and headline) else make()
    if args.iterations and headline:
        w.iterations = args.iterations
    B, n = w.target.shape
    tdtype = torch.float64 if w.dtype == np.float64 else torch.float32
    ws = np.dtype(w.dtype).itemsize
    values, root = weighted_values(w)
    plan = Plan(w.n, w.me, w.rows_total - w.me, w.indptr, w.indices, values,
                dtype=tdtype, accelerated=w.accelerated, device="cuda:0")
    if root is not None:
        plan.set_metric(root)
    m = plan.m
    dev = torch.device("cuda:0")
    target = torch.as_tensor(w.target, device=dev)
    rhs = torch.as_tensor(np.tile(w.rhs, (B, 1)).astype(w.dtype), device=dev)
    kw = dict(max_iterations=w.iterations, early_stop=False, shared_bounds=True)

    for _ in range(warmup):
        plan.project(target, rhs, **kw)
    ms_per_step, out = time_calls(torch, lambda: plan.project(target, rhs, **kw), steps)
    value = B / (ms_per_step / 1e3)
    status = out.status.cpu().numpy()

    # instrumented replay: HIP events around the iteration kernels' launches
    plan.project(target, rhs, timing=True, **kw)
    torch.cuda.synchronize()
    tm = plan.last_timing()
    iters = max(int(tm["iterations"]), 1)
    if tm["linear_kybar"]:
        # K ybar formed from K y: the row pass gathers y (n), reads d, r and the
        # previous K y (3m), writes d and K y (2m); the column pass gathers d+ (m),
        # reads y, yhat (2n) and writes y (n), with no ybar vector
        bytes_row = B * ws * (n + 5 * m)
        bytes_col = B * ws * (3 * n + m)
    else:
        bytes_row = B * ws * (n + 3 * m)    # gather ybar (n), read d, r (2m), write d (m)
        bytes_col = B * ws * (4 * n + m)    # gather d+ (m), read y, yhat (2n), write y, ybar (2n)
    bytes_iter = B * ws * (5 * n + 3 * m)   # the per-iteration contract figure
    iter_ms = tm["loop_ms"] / iters
    if tm["resident"]:
        # one launch runs every iteration with the state on chip
        dominant, dom_bytes, dom_ms = "k_resident", bytes_iter * iters, tm["loop_ms"]
        row_ms = col_ms = None
    else:
        row_ms, col_ms = tm["row_ms"] / iters, tm["col_ms"] / iters
        # a quarter wavefront per column (k_col_pass_q) where the wide tile's
        # gathered slice of d+ exceeds an XCD's L2
        col_kernel = "k_col_pass_q" if tm["narrow_columns"] else "k_col_pass"
        dominant = col_kernel if col_ms >= row_ms else "k_row_pass"
        dom_bytes, dom_ms = (bytes_col, col_ms) if dominant == col_kernel else (bytes_row, row_ms)
    achieved = dom_bytes / (dom_ms / 1e3) / 1e9
    traffic = traffic_from_profiles(config, dominant, B, w.iterations)
    if tm["resident"]:
        # The iterate stays on chip: what the launch moves is the shared matrix's
        # chunk streams from L2 (every tile re-reads them each iteration) and the
        # LDS gathers.  Price it against the probes' ceilings at the same shape.
        info = plan.info
        # samples per workgroup: 16 bytes of samples per LDS entry (2 fp64, 4
        # fp32), or 8 fp32 in two LDS planes where n, m <= 1024
        bt = int(info.resident_tile_samples)
        pad = 64 * (2 if ws == 8 else 4)                # the batch's padding unit
        tiles = -(-B // pad) * pad // bt                # the padded batch's tiles
        l2_bytes = tiles * iters * int(info.resident_stream_bytes)
        entries = int(info.resident_stream_bytes) // (12 if ws == 8 else 8)
        planes = bt * ws // 16                          # 16-byte LDS reads per gathered entry
        lds_iter = 16 * planes * (entries + 2 * int(info.resident_row_slots)
                                  + int(info.resident_col_slots))
        lds_launch = tiles * iters * lds_iter
        lds_alloc = (n + 1 + m + 1) * 16 if planes == 1 else 2 * 32800
        ceil = probe_ceilings(torch, tiles, lds_alloc, int(info.resident_stream_bytes))
        l2_rate = l2_bytes / (dom_ms / 1e3) / 1e9
        lds_rate = lds_launch / (dom_ms / 1e3) / 1e9
        roofline = {
            "bound": "l2",
            "kernel": dominant,
            "achieved": l2_rate,
            "peak": ceil["l2"]["GBs"],
            "unit": "GB/s",
            "frac": l2_rate / ceil["l2"]["GBs"],
            "traffic": traffic,
            "bytes_per_launch": l2_bytes,
            "avg_launch_ms": dom_ms,
            "what": "L2 -> CU bytes of the shared matrix's chunk streams: "
                    f"{int(info.resident_stream_bytes)} B per workgroup per iteration x "
                    f"{tiles} workgroups x {iters} iterations",
            "peak_source": "measured in this run: best rate of the k_probe_stream ceiling probe "
                           f"(libpurin_probe.so) at {tiles} workgroups of 1024 threads, "
                           f"{ceil['wave_chunks']} 3072-byte chunks per wavefront per pass, "
                           f"{ceil['l2']['unroll']} in flight, {ceil['l2']['lds_bytes']} B LDS",
            "lds": {"achieved": lds_rate, "peak": ceil["lds"]["GBs"],
                    "frac": lds_rate / ceil["lds"]["GBs"], "bytes_per_launch": lds_launch,
                    "what": f"{16 * planes} B per gathered entry ({entries} per workgroup "
                            "per iteration, padding included) + the slots' own entries (2 per "
                            "row, 1 per column)",
                    "peak_source": "measured in this run: best rate of k_probe_lds "
                                   "(conflict-free ds_read_b128)"},
            "hbm": {"achieved": achieved, "peak": HBM_PEAK_GBS, "frac": achieved / HBM_PEAK_GBS,
                    "bytes_per_launch": dom_bytes,
                    "note": "algorithmic state bytes B*ws*(5n+3m) per iteration; they stay "
                            "on chip, so this exceeds the HBM peak and does not bound the "
                            "kernel (context only)"},
            "probes": {"l2": ceil["l2_all"], "lds": ceil["lds_all"]},
        }
    else:
        roofline = {
            "bound": "hbm",
            "kernel": dominant,
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic,
            "bytes_per_launch": dom_bytes,
            "avg_launch_ms": dom_ms,
            "what": (f"algorithmic bytes of one {dominant} launch (one pass of one "
                     "iteration): "
                     + ("K ybar formed from K y (no ybar stream; the row pass reads and "
                        "writes K y)" if tm["linear_kybar"] else "ybar streamed")),
        }
    # the streaming two-pass path on the same inputs, for comparison
    streaming_ms = None
    if headline and tm["resident"] and not args.no_streaming:
        streaming_ms, _ = time_calls(
            torch, lambda: plan.project(target, rhs, streaming=True, **kw), 1)

    line = {
        "metric": METRICS[config],
        "value": value,
        "unit": "projections/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64" if ws == 8 else "f32",
        "data": f"synthetic ({w.name} generator, numpy default_rng seed {config})",
        "config": {
            "workload": {
                2: "config2: n=4096, 1024 eq + 2048 ineq rows x 8 cols, 8192 bound rows, "
                   "batch 1024, fp64, accelerated CP, fixed iterations, full projection",
                3: "config3: node-edge incidence of 10000 nodes x 40000 edges (eq rows), "
                   "edge bounds [0, U(1,5)], WeightedDistance D~U(0.5,2), batch 256, fp64, "
                   "fixed-step CP, fixed iterations, full projection",
                4: "config4: n=1024, 256 eq + 512 ineq rows x 16 cols, bounds [-2,2], "
                   "batch 65536, fp32, accelerated CP, fixed iterations, full projection",
            }[config],
            "n": n, "kept_rows": m, "bound_rows": int(plan.info.bound_rows),
            "nnz_kept": int(plan.info.nnz_kept), "batch": B, "iterations": w.iterations,
            "parallelism": "1 GPU (batch-parallel)",
        },
        "roofline": roofline,
        "iteration": {
            "cp_iterations_per_s": w.iterations * 1e3 / ms_per_step,
            "resident_kernel": bool(tm["resident"]),
            "linear_kybar": bool(tm["linear_kybar"]),
            "narrow_columns": bool(tm["narrow_columns"]),
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
    if headline:
        # per-sample bounds: the kernels of a caller whose bound rows depend on theta
        kw_ps = dict(kw, shared_bounds=False)
        plan.project(target, rhs, **kw_ps)
        ps_ms, ps_out = time_calls(torch, lambda: plan.project(target, rhs, **kw_ps), steps)
        line["per_sample_bounds"] = {
            "ms_per_step": ps_ms,
            "value": B / (ps_ms / 1e3),
            "unit": "projections/s",
            "y_bit_identical_to_shared": bool(torch.equal(ps_out.y, out.y)),
            "what": "the same purin_cp_project call with shared_bounds = 0 (lower/upper read "
                    "per sample: the kernels of bound rows whose rhs depends on theta)",
        }
        # the PURIN-API front end on the same problem (constant bound rows: it
        # selects the shared-bounds kernels by itself)
        line["purin_api"] = purin_api_timing(torch, w, values, root, target, steps)
    ctx = dict(w=w, plan=plan, target=target, rhs=rhs, kw=kw, B=B, n=n, m=m, ws=ws, dev=dev)
    return line, ctx


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", type=int, default=2, choices=(2, 3, 4))
    ap.add_argument("--mode", default="project", choices=("project", "values", "qp", "dense"),
                    help="project: the headline (default); values / qp / dense: the widened "
                         "paths (per-sample coefficients, diagonal QP, dense adapter)")
    ap.add_argument("--batch", type=int, default=None)
    ap.add_argument("--iterations", type=int, default=None)
    ap.add_argument("--cpu-samples", type=int, default=None,
                    help="samples of the all-core CPU baseline leg")
    ap.add_argument("--cpu-samples-one", type=int, default=None,
                    help="samples of the one-core CPU baseline leg")
    ap.add_argument("--cpu-adjoint-samples", type=int, default=32,
                    help="samples of the one-thread CPU adjoint leg (config2)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-adjoint", action="store_true", help="skip the adjoint leg (config2)")
    ap.add_argument("--no-others", action="store_true",
                    help="skip the config3 / config4 sub-objects of the default (config2) line")
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

    if args.mode != "project":
        run_mode(args, torch)
        return

    line, ctx = measure(args, torch, args.config, steps=args.steps, warmup=args.warmup,
                        headline=True)
    w, plan, target, rhs, kw = ctx["w"], ctx["plan"], ctx["target"], ctx["rhs"], ctx["kw"]
    B, n, m, ws, dev = ctx["B"], ctx["n"], ctx["m"], ctx["ws"], ctx["dev"]
    adjoint_leg = args.config == 2 and not args.no_adjoint

    if adjoint_leg:
        cot = torch.as_tensor(np.random.default_rng(5).normal(0.0, 1.0, (B, n)), device=dev)
        fwd = plan.project(target, rhs, save=True, **kw)
        adj = dict(force_eligible=True)
        plan.adjoint(fwd.saved, None, None, cot, **adj)       # warmup
        adj_ms, res = time_calls(torch, lambda: plan.adjoint(fwd.saved, None, None, cot, **adj),
                                 max(1, min(args.steps, 3)))
        stats = plan.last_adjoint_stats()
        width = 2 * n + m
        abytes = adjoint_bytes(B, ws, width, stats["arnoldi_steps"], 30)
        sbytes = adjoint_streamed_bytes(B, ws, n, m, stats["arnoldi_steps"], 30)
        info = res.info.cpu().numpy()
        line["adjoint"] = {
            "workload": "config5: VJP w.r.t. y_hat and (b, h) on the config2 problem, cotangent "
                        "N(0,1) seed 5, GMRES restart 30, max 100, tol 1e-9, at the "
                        f"{w.iterations}-iteration state with gradient eligibility forced on",
            "ms_per_vjp_batch": adj_ms,
            "vjps_per_s": B / (adj_ms / 1e3),
            "arnoldi_steps": stats["arnoldi_steps"],
            "cycles": stats["cycles"],
            "gmres_info": {str(k): int(v) for k, v in zip(*np.unique(info, return_counts=True))},
            "algorithmic_bytes": abytes,
            "achieved_GBs": abytes / (adj_ms / 1e3) / 1e9,
            "frac_of_hbm_peak": abytes / (adj_ms / 1e3) / 1e9 / HBM_PEAK_GBS,
            "streamed_bytes": sbytes,
            "streamed_GBs": sbytes / (adj_ms / 1e3) / 1e9,
            "streamed_frac_of_hbm_peak": sbytes / (adj_ms / 1e3) / 1e9 / HBM_PEAK_GBS,
        }
        # config5 as stated: the forward run to convergence (tolerance 1e-9, up to
        # 10000 iterations: the reference's defaults) and the VJP at that solution,
        # each timed on its own; eligibility comes from the forward
        kc = dict(kw, max_iterations=10000, early_stop=True, tolerance=1e-9)
        plan.project(target, rhs, save=True, **kc)                    # warmup
        f_ms, fwd_c = time_calls(torch, lambda: plan.project(target, rhs, save=True, **kc), 1)
        plan.adjoint(fwd_c.saved, None, None, cot)                     # warmup
        a_ms, res_c = time_calls(torch, lambda: plan.adjoint(fwd_c.saved, None, None, cot), 1)
        stats_c = plan.last_adjoint_stats()
        st_c = fwd_c.status.cpu().numpy()
        it_c = fwd_c.iterations.cpu().numpy()
        info_c = res_c.info.cpu().numpy()
        line["adjoint_converged"] = {
            "workload": "config5: the config2 problem solved to convergence (early stop, tol 1e-9, "
                        "at most 10000 accelerated iterations), then the VJP w.r.t. y_hat and "
                        "(b, h) at that solution (cotangent N(0,1) seed 5, GMRES restart 30, "
                        "max 100, tol 1e-9), eligibility from the forward",
            "forward_ms": f_ms,
            "forward_statuses": {str(k): int(v) for k, v in zip(*np.unique(st_c, return_counts=True))},
            "forward_iterations_max": int(it_c.max()),
            "forward_iterations_mean": float(it_c.mean()),
            "adjoint_ms": a_ms,
            "vjps_per_s": B / (a_ms / 1e3),
            "eligible": int(fwd_c.eligible.sum().item()),
            "valid": int(res_c.valid.sum().item()),
            "arnoldi_steps": stats_c["arnoldi_steps"],
            "cycles": stats_c["cycles"],
            "gmres_info": {str(k): int(v) for k, v in zip(*np.unique(info_c, return_counts=True))},
        }

    if not args.no_cpu:
        default_sample = CPU_SAMPLES[args.config]
        one = args.cpu_samples_one or default_sample[0]
        full = args.cpu_samples or default_sample[1]
        line["cpu_baseline"] = cpu_baseline(w, min(one, B), min(full, B))
        if adjoint_leg:
            # the checker's adjoint on the first samples, linearised at the GPU's
            # forward state of the same samples (samples are independent)
            from oracle import projection as op

            k = min(args.cpu_adjoint_samples, B)
            cfg = op.Config(accelerated=True, max_iterations=w.iterations, early_stop=False)
            one_c = op.Canonical(n=w.n, me=w.me, rows=w.rows(), coef=w.coefs())
            pre = op.presolve(one_c, w.rhs[None, :], cfg, np.float64)
            rhs_k = np.tile(pre.kept_rhs, (k, 1))
            w.cotangent = np.random.default_rng(5).normal(0.0, 1.0, (B, n))
            st = plan.solve(rhs_k, w.target[:k], pre.lower[0], pre.upper[0],
                            max_iterations=w.iterations, early_stop=False, shared_bounds=True)
            line["cpu_baseline_adjoint"] = cpu_baseline_adjoint(
                w, plan, st.y.cpu().numpy(), st.dual.cpu().numpy(), pre.lower[0], pre.upper[0],
                rhs_k, k)
    # the other BASELINE configurations, each timed on its own plan after the
    # headline's legs (3 steps after one warm-up call)
    if args.config == 2 and not args.no_others and not args.batch and not args.iterations:
        del ctx, plan, target, rhs
        torch.cuda.empty_cache()
        for c in (3, 4):
            print(f"bench: config{c}", file=sys.stderr, flush=True)
            sub, sctx = measure(args, torch, c, steps=max(1, min(args.steps, 3)), warmup=1,
                                headline=False)
            for k in ("n_gpus", "higher_is_better", "scaling", "vs_baseline"):
                sub.pop(k, None)
            if not args.no_cpu:
                one, full = CPU_SAMPLES_OTHER[c]
                sub["cpu_baseline"] = cpu_baseline(sctx["w"], one, full)
            line[f"config{c}"] = sub
            del sctx
            torch.cuda.empty_cache()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
