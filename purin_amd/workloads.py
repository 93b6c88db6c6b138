"""Seeded synthetic problems for the benchmark configurations.

Each generator draws, with ``numpy.random.default_rng(seed)``, in this order:
the constraint rows (equalities, then inequalities: sorted distinct columns,
then their values), the feasible point ``x0``, the inequality slack, then the
candidates ``yhat``.  Variable bounds are singleton inequality rows appended
after the general inequalities: all upper rows ``+y_j <= U_j`` first, then all
lower rows ``-y_j <= -L_j`` (the row order of ``ParametricQP.from_bounds``,
reference src/purin/problems/qp.py:308-398).

Rows are returned as one CSR matrix over all ``me + mi`` canonical rows with
right-hand side ``rhs`` such that ``K[:me] y = rhs[:me]``, ``K[me:] y <= rhs[me:]``
(the sign convention of reference src/purin/problems/expressions.py:298-309).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


@dataclass
class Workload:
    name: str
    n: int
    me: int
    indptr: np.ndarray
    indices: np.ndarray
    data: np.ndarray
    rhs: np.ndarray            # (me+mi,) shared by the batch
    target: np.ndarray         # (B, n)
    dtype: object
    accelerated: bool
    iterations: int
    metric: np.ndarray | None = None
    cotangent: np.ndarray | None = None
    info: dict = field(default_factory=dict)

    @property
    def rows_total(self):
        return self.indptr.size - 1

    @property
    def batch(self):
        return self.target.shape[0]

    def dense(self):
        out = np.zeros((self.rows_total, self.n))
        for i in range(self.rows_total):
            s, e = self.indptr[i], self.indptr[i + 1]
            out[i, self.indices[s:e]] = self.data[s:e]
        return out

    def rows(self):
        return [self.indices[self.indptr[i]:self.indptr[i + 1]].tolist()
                for i in range(self.rows_total)]

    def coefs(self):
        return [self.data[self.indptr[i]:self.indptr[i + 1]].tolist()
                for i in range(self.rows_total)]


def _csr_from_rows(rows, vals):
    indptr = np.zeros(len(rows) + 1, np.int64)
    indptr[1:] = np.cumsum([len(r) for r in rows])
    indices = np.concatenate([np.asarray(r, np.int64) for r in rows]) if rows else np.zeros(0, np.int64)
    data = np.concatenate([np.asarray(v, np.float64) for v in vals]) if rows else np.zeros(0)
    return indptr, indices.astype(np.int32), data


def _append_bounds(rows, vals, rhs, lower, upper):
    n = lower.size
    for j in range(n):
        if np.isfinite(upper[j]):
            rows.append([j]); vals.append([1.0]); rhs.append(upper[j])
    for j in range(n):
        if np.isfinite(lower[j]):
            rows.append([j]); vals.append([-1.0]); rhs.append(-lower[j])


def random_rows(*, seed, n, me, mi, width, value_sd, x0_half, bound, batch, target_sd,
                dtype, accelerated, iterations, name, extra_draw_cot=False):
    """Random sparse rows with a feasible point; configs 1, 2 and 4."""
    rng = np.random.default_rng(seed)
    rows, vals = [], []
    for _ in range(me + mi):
        cols = np.sort(rng.choice(n, width, replace=False))
        rows.append(cols.tolist())
        vals.append(rng.normal(0.0, value_sd, width).tolist())
    x0 = rng.uniform(-x0_half, x0_half, n)
    K = np.zeros((me + mi, n))
    for i, (c, v) in enumerate(zip(rows, vals)):
        K[i, c] = v
    b = K[:me] @ x0
    h = K[me:] @ x0 + rng.uniform(0.0, 1.0, mi)
    rhs = list(b) + list(h)
    _append_bounds(rows, vals, rhs, np.full(n, -bound), np.full(n, bound))
    target = rng.normal(0.0, target_sd, (batch, n))
    indptr, indices, data = _csr_from_rows(rows, vals)
    return Workload(name, n, me, indptr, indices, data, np.asarray(rhs), target.astype(dtype),
                    np.dtype(dtype), accelerated, iterations,
                    info=dict(mi_general=mi, width=width, bound=bound))


def ragged_rows(seed, *, n, me, mi, wmin, wmax, batch, bound=1.0, dtype=np.float64,
                accelerated=False, iterations=200, target_sd=2.0):
    """Random sparse rows of ragged widths (uniform in [wmin, wmax], wmin >= 2 so
    no general row is a singleton) with a feasible point, for parity tests of
    schedules whose slots hold rows and columns of unequal length."""
    rng = np.random.default_rng(seed)
    rows, vals = [], []
    for _ in range(me + mi):
        w = int(rng.integers(wmin, wmax + 1))
        rows.append(np.sort(rng.choice(n, w, replace=False)).tolist())
        vals.append(rng.normal(0.0, 1.0, w).tolist())
    x0 = rng.uniform(-0.5 * bound, 0.5 * bound, n)
    Kx = np.array([np.dot(v, x0[c]) for c, v in zip(rows, vals)])
    rhs = list(Kx[:me]) + list(Kx[me:] + rng.uniform(0.0, 1.0, mi))
    _append_bounds(rows, vals, rhs, np.full(n, -bound), np.full(n, bound))
    target = rng.normal(0.0, target_sd, (batch, n))
    indptr, indices, data = _csr_from_rows(rows, vals)
    return Workload(f"ragged{seed}", n, me, indptr, indices, data, np.asarray(rhs),
                    target.astype(dtype), np.dtype(dtype), accelerated, iterations,
                    info=dict(mi_general=mi, width=(wmin, wmax), bound=bound))


def config1(batch=32):
    """Plumbing: n=64, 16 eq + 32 ineq rows of 4 columns, fp64, fixed-step, 1000 iterations."""
    return random_rows(seed=1, n=64, me=16, mi=32, width=4, value_sd=1.0, x0_half=0.5,
                       bound=1.0, batch=batch, target_sd=2.0, dtype=np.float64,
                       accelerated=False, iterations=1000, name="config1")


def config2(batch=1024):
    """Mid fp64: n=4096, 1024 eq + 2048 ineq rows of 8 columns, accelerated, 2000 iterations."""
    return random_rows(seed=2, n=4096, me=1024, mi=2048, width=8, value_sd=1.0, x0_half=0.5,
                       bound=1.0, batch=batch, target_sd=2.0, dtype=np.float64,
                       accelerated=True, iterations=2000, name="config2")


def config4(batch=65536):
    """High-batch fp32: n=1024, 256 eq + 512 ineq rows of 16 columns, accelerated, 500 iterations."""
    return random_rows(seed=4, n=1024, me=256, mi=512, width=16, value_sd=0.25, x0_half=1.0,
                       bound=2.0, batch=batch, target_sd=3.0, dtype=np.float32,
                       accelerated=True, iterations=500, name="config4")


def config3(batch=256, nodes=10000, edges=40000):
    """Network-flow conservation, WeightedDistance metric, fp64, fixed-step, 3000 iterations."""
    rng = np.random.default_rng(3)
    ends = np.empty((edges, 2), np.int64)
    for e in range(edges):
        ends[e] = rng.choice(nodes, 2, replace=False)
    b = rng.normal(0.0, 1.0, nodes)
    b -= b.mean()
    U = rng.uniform(1.0, 5.0, edges)
    D = rng.uniform(0.5, 2.0, edges)
    target = rng.normal(0.0, 1.0, (batch, edges))
    node_rows = [[] for _ in range(nodes)]
    for e in range(edges):
        u, v = ends[e]
        node_rows[u].append((e, 1.0))
        node_rows[v].append((e, -1.0))
    rows = [[c for c, _ in sorted(r)] for r in node_rows]
    vals = [[x for _, x in sorted(r)] for r in node_rows]
    rhs = list(b)
    _append_bounds(rows, vals, rhs, np.zeros(edges), U)
    indptr, indices, data = _csr_from_rows(rows, vals)
    return Workload("config3", edges, nodes, indptr, indices, data, np.asarray(rhs), target,
                    np.dtype(np.float64), False, 3000, metric=D,
                    info=dict(mi_general=0, nodes=nodes))


def config5(batch=1024):
    """Adjoint on the config-2 problem with N(0,1) cotangents drawn from seed 5."""
    w = config2(batch)
    w.name = "config5"
    w.cotangent = np.random.default_rng(5).normal(0.0, 1.0, (batch, w.n))
    return w


def small_random(seed, *, n, me, mi, width, batch, bound=1.0, dtype=np.float64,
                 accelerated=False, iterations=200, target_sd=2.0):
    """Scaled-down version of the random-row configs for parity tests."""
    return random_rows(seed=seed, n=n, me=me, mi=mi, width=width, value_sd=1.0, x0_half=0.5,
                       bound=bound, batch=batch, target_sd=target_sd, dtype=dtype,
                       accelerated=accelerated, iterations=iterations, name=f"small{seed}")
