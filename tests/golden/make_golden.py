"""Write tests/golden/config1.npz: the plumbing configuration's inputs and the
oracle's outputs, committed as fixtures.

config1 (the reference-runnable CPU case): n = 64, 16 equality + 32 inequality
rows of 4 columns, bounds [-1, 1] as 128 singleton rows, batch 32, seed 1.

Contents
  inputs   indptr, indices, data (CSR of all 176 rows), rhs (176,), target (32, 64),
           cot (32, 64) cotangent N(0, 1) from seed 5
  fixed    1000 fixed iterations, fixed-step CP (the configuration as stated), in
           float64 (f64_*) and float32 (f32_*): y, multipliers, slacks, status,
           iterations, residual
  conv     to convergence (tolerance 1e-9, up to 10000 iterations, early stop) in
           float64: y, status, iterations, and the VJP of y w.r.t. target and
           rhs for ``cot`` (default GMRES settings) -- conv_*

The reference is JAX (absent here), so these are the oracle's outputs; the
oracle itself is pinned by the reference's known-answer tests and by exact QP
solutions (tests/test_oracle_*.py).  Run from the repository root:
    python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import projection as op  # noqa: E402
from purin_amd import workloads  # noqa: E402

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "config1.npz")
FIXED_ITERATIONS = 1000


def compute():
    w = workloads.config1(batch=32)
    canon = op.Canonical(n=w.n, me=w.me, rows=w.rows(), coef=w.coefs())
    B = w.target.shape[0]
    rhs = np.tile(w.rhs, (B, 1))
    cot = np.random.default_rng(5).normal(0.0, 1.0, (B, w.n))
    out = dict(indptr=w.indptr.astype(np.int64), indices=w.indices.astype(np.int32),
               data=w.data.astype(np.float64), rhs=np.asarray(w.rhs, np.float64),
               target=w.target.astype(np.float64), cot=cot, me=np.int64(w.me),
               mi=np.int64(w.rows_total - w.me))
    for tag, dtype in (("f64", np.float64), ("f32", np.float32)):
        cfg = op.Config(accelerated=False, max_iterations=FIXED_ITERATIONS, early_stop=False)
        r = op.solve(canon, w.target.astype(dtype), rhs.astype(dtype), cfg, dtype=dtype)
        out[f"{tag}_y"] = r.y
        out[f"{tag}_multipliers"] = np.concatenate((r.multipliers_eq, r.multipliers_ineq), axis=1)
        out[f"{tag}_slacks"] = r.slacks
        out[f"{tag}_status"] = np.asarray(r.status, np.int32)
        out[f"{tag}_iterations"] = np.asarray(r.iterations, np.int32)
        out[f"{tag}_residual"] = r.residual_inf_norm
    cfg = op.Config(accelerated=False, max_iterations=10000, tolerance=1e-9)
    res, g_target, g_rhs, adj = op.vjp(canon, w.target, rhs, cfg, cot)
    out.update(conv_y=res.y, conv_status=np.asarray(res.status, np.int32),
               conv_iterations=np.asarray(res.iterations, np.int32),
               conv_eligible=np.asarray(res.gradient_eligible, bool),
               conv_valid=np.asarray(adj.valid, bool), conv_g_target=g_target, conv_g_rhs=g_rhs)
    return out


def main():
    np.savez_compressed(PATH, **compute())
    print(f"wrote {PATH}")


if __name__ == "__main__":
    main()
