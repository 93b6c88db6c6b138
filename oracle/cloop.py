"""ctypes front of ``oracle/cp_loop.c``: the fixed-iteration CP loop in plain C.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): the CPU-baseline timing
of ``bench.py`` and its pinning test (tests/test_oracle_cloop.py) use it.

The set-up (bound presolve, row scaling, initial steps) is the NumPy oracle's
(``oracle.projection.presolve``, ``oracle.cp.step_sizes``); only the iteration
loop, where the time goes, runs in C.  Pinned by: equality with
``oracle.cp.sparse_cp(..., early_stop=False)`` on the same inputs.
"""

from __future__ import annotations

import ctypes as C
import os
import subprocess
import time

import numpy as np

from oracle import cp as _cp
from oracle import projection as _op

HERE = os.path.dirname(os.path.abspath(__file__))
SOURCE = os.path.join(HERE, "cp_loop.c")
LIB_PATH = os.path.join(HERE, "libcp_loop.so")
CFLAGS = ["-O3", "-march=x86-64-v3", "-ffp-contract=off", "-fopenmp", "-shared", "-fPIC",
          "-Wall", "-Wextra"]

_lib = None


def build(cc="gcc"):
    """Compile ``cp_loop.c`` into ``oracle/libcp_loop.so`` (no FMA contraction, so each
    operation rounds like the NumPy oracle's)."""
    tmp = LIB_PATH + ".tmp"
    subprocess.run([cc, *CFLAGS, SOURCE, "-o", tmp, "-lm"], check=True)
    os.replace(tmp, LIB_PATH)


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: run oracle.cloop.build()")
        lib = C.CDLL(LIB_PATH)
        for suffix in ("f64", "f32"):
            fn = getattr(lib, f"purin_oracle_cp_fixed_{suffix}")
            fn.restype = C.c_int
            fn.argtypes = ([C.c_int64] * 3 + [C.c_void_p] * 3 + [C.c_int64] + [C.c_void_p] * 7
                           + [C.c_int64, C.c_int, C.c_int, C.c_void_p, C.c_void_p])
        _lib = lib
    return _lib


def _p(a):
    return None if a is None else C.c_void_p(a.ctypes.data)


def prepare(canon, target, rhs, cfg, dtype=np.float64):
    """The oracle's set-up of ``BoundProjection.solve`` up to the loop (bounds.py:192-236,
    kernels.py:209-227): shared scaled CSR of the kept rows, per-sample inputs, steps."""
    dtype = np.dtype(dtype)
    target = np.ascontiguousarray(target, dtype)
    rhs = np.asarray(rhs, dtype)
    pre = _op.presolve(canon, rhs, cfg, dtype)
    support, mask = pre.support[pre.rows], pre.mask[pre.rows]
    values = np.ascontiguousarray(pre.kept_values[0])
    tau, sigma = _cp.step_sizes(np.ones_like(target), pre.kept_values, support, mask,
                                accelerated=cfg.accelerated, safety=cfg.safety,
                                norm_bound_flag=cfg.norm_bound,
                                diagonal_preconditioning=cfg.diagonal_preconditioning,
                                norm_iterations=cfg.norm_iterations, norm_seed=cfg.norm_seed)
    counts = mask.sum(axis=1)
    rptr = np.concatenate(([0], np.cumsum(counts))).astype(np.int64)
    ridx = np.ascontiguousarray(support[mask], np.int32)
    rval = np.ascontiguousarray(values[mask], dtype)
    return dict(n=canon.n, m=len(pre.rows), me=canon.me, rptr=rptr, ridx=ridx, rval=rval,
                rhs=np.ascontiguousarray(pre.kept_rhs, dtype), target=target,
                lower=np.ascontiguousarray(pre.lower, dtype),
                upper=np.ascontiguousarray(pre.upper, dtype),
                tau=np.ascontiguousarray(np.broadcast_to(tau, target.shape[:1]), dtype),
                sigma=np.ascontiguousarray(np.broadcast_to(sigma, target.shape[:1]), dtype),
                dtype=dtype)


def run(prep, iterations, accelerated, threads=1, dual0=None):
    """Run the C loop; returns ``(y, d, seconds)``."""
    lib = load()
    dtype = prep["dtype"]
    fn = lib.purin_oracle_cp_fixed_f64 if dtype == np.float64 else lib.purin_oracle_cp_fixed_f32
    batch, n = prep["target"].shape
    m = prep["m"]
    y = np.empty((batch, n), dtype)
    d = np.empty((batch, m), dtype)
    d0 = None if dual0 is None else np.ascontiguousarray(dual0, dtype)
    t0 = time.perf_counter()
    rc = fn(n, m, prep["me"], _p(prep["rptr"]), _p(prep["ridx"]), _p(prep["rval"]), batch,
            _p(prep["rhs"]), _p(prep["target"]), _p(prep["lower"]), _p(prep["upper"]), _p(d0),
            _p(prep["tau"]), _p(prep["sigma"]), int(iterations), int(bool(accelerated)),
            int(threads), _p(y), _p(d))
    dt = time.perf_counter() - t0
    if rc:
        raise MemoryError("cp_loop scratch allocation failed")
    return y, d, dt
