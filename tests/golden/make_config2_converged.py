"""Write tests/golden/config2_converged.npz: the oracle's early-stop solve of
three config2 samples at the reference's default stopping rule.

config2 (n = 4096, 1024 equality + 2048 inequality rows of 8 columns, bounds
[-1, 1] as 8192 singleton rows, seed 2), accelerated CP with the default
tolerance 1e-9 and at most 10000 iterations, early stop on (the reference's
loop, src/purin/solvers/chambolle_pock/kernels.py:228-305, with the bound
presolve of bounds.py:170-317).  The samples are 0, 511 and 1023 of the
generator's batch of 1024.  The config5 adjoint is taken at this forward: a
sample the forward does not converge gets no gradient (bounds.py:148-153).

Contents
  samples     (3,) batch indices
  status      (3,) 0 converged, 1 iteration limit
  iterations  (3,)
  residual    (3,) residual_inf_norm in original units
  y           (3, 4096) the iterate returned

The reference is JAX (absent here), so these are the oracle's outputs; the
oracle is pinned by the reference's known-answer tests and by exact QP
solutions (tests/test_oracle_*.py).  Takes about two minutes.  Run from the
repository root:
    python tests/golden/make_config2_converged.py
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

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "config2_converged.npz")
SAMPLES = np.array([0, 511, 1023])
TOLERANCE = 1e-9
MAX_ITERATIONS = 10000


def main():
    w = workloads.config2()
    canon = op.Canonical(n=w.n, me=w.me, rows=w.rows(), coef=w.coefs())
    cfg = op.Config(accelerated=True, max_iterations=MAX_ITERATIONS, tolerance=TOLERANCE,
                    early_stop=True)
    res = op.solve(canon, w.target[SAMPLES], np.tile(w.rhs, (len(SAMPLES), 1)), cfg)
    np.savez_compressed(PATH, samples=SAMPLES, status=np.asarray(res.status),
                        iterations=np.asarray(res.iterations),
                        residual=np.asarray(res.residual_inf_norm), y=np.asarray(res.y))
    print(f"wrote {PATH}: status {res.status}, iterations {res.iterations}, "
          f"residual {res.residual_inf_norm}")


if __name__ == "__main__":
    main()
