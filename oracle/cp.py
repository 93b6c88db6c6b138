"""NumPy restatement of PURIN's sparse Chambolle--Pock (CP) kernels.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): the checker for the HIP
path, never imported by the product.

Every function follows a reference file:line (paths relative to the reference
repository root, ``src/purin/...``).  Arrays are batch-major ``(B, .)`` like the
reference.  The arithmetic is done in the dtype of the inputs (float32 or
float64) so that fp32 runs round like the reference's fp32 runs.

What pins each function (besides being a line-by-line restatement):

* ``layout``/``matvec``/``tmatvec``: dense ``einsum`` (tests/test_oracle_cp.py,
  mirroring tests/test_sparse_layouts.py:17-51 of the reference).
* ``proximal_coefficients``/``cp_step``: the closed form
  ``(y - tau(2y + c))/(1 + tau q)`` to 1e-14 and cached == uncached bit equality
  (reference tests/test_regression_cp_proximal_coefficients.py:11-53).
* ``norm_bound_steps``: closed form ``sqrt(max rowsum * max colsum)``.
* ``diagonal_step_sizes``: the bound ``||sqrt(S) K sqrt(T)||_2 <= safety``
  (reference tests/test_regression_cp_diagonal_steps.py:13-26).
* ``sparse_cp``/``diagnostics``: converged outputs equal the exact QP solution
  from brute-force active-set enumeration (``oracle/qp.py``) and satisfy KKT.
* ``norm_estimate``: its start vector is this build's own deterministic
  generator (the reference draws it from ``jax.random``, which is absent here);
  the estimate is pinned against ``numpy.linalg.norm(K, 2)`` from below and the
  converged adjoint does not depend on it (fixed-point invariance).
"""

from __future__ import annotations

from typing import NamedTuple

import numpy as np


class CPOutput(NamedTuple):
    """kernels.py:15-23."""

    y: np.ndarray
    dual: np.ndarray
    iterations: np.ndarray
    residual: np.ndarray
    gap: np.ndarray
    converged: np.ndarray


# ---------------------------------------------------------------------------
# sparse layout and products
# ---------------------------------------------------------------------------


def layout(rows, n):
    """Padded ELL support/mask; kernels.py:26-40."""
    rows = [tuple(int(c) for c in r) for r in rows]
    width = max(1, max(map(len, rows), default=0))
    support = np.zeros((len(rows), width), dtype=np.int32)
    mask = np.zeros_like(support, dtype=bool)
    for i, row in enumerate(rows):
        support[i, : len(row)] = row
        mask[i, : len(row)] = True
    return support, mask


def ell_values(matrix, support, mask):
    """Coefficient values of a dense matrix on an ELL support (zero when masked)."""
    matrix = np.asarray(matrix)
    rows = np.arange(support.shape[0])[:, None]
    return np.where(mask, matrix[rows, support], 0).astype(matrix.dtype)


def matvec(values, support, mask, x):
    """``(Kx)_bi = sum_s mask*values*x[b, support]`` in slot order.

    linalg/sparse/operators.py:507-518 (shared ``(m,w)`` or batched ``(B,m,w)``
    coefficients).
    """
    batch = x.shape[0]
    if support.shape[0] == 0:
        return np.empty((batch, 0), dtype=x.dtype)
    coeff = values if values.ndim == 3 else values[None, :, :]
    gathered = x[:, support]
    prod = np.where(mask[None, :, :], coeff * gathered, x.dtype.type(0))
    acc = prod[:, :, 0].copy()
    for s in range(1, prod.shape[2]):
        acc = acc + prod[:, :, s]
    return acc


def tmatvec(values, support, mask, v, n):
    """Scatter-add ``K^T v``; linalg/sparse/operators.py:521-533.

    The accumulation order is row-major over ``(row, slot)``, i.e. increasing
    row index per column (the CSC order the HIP gather uses).
    """
    batch = v.shape[0]
    out = np.zeros((batch, n), dtype=v.dtype)
    if support.shape[0] == 0:
        return out
    coeff = values if values.ndim == 3 else np.broadcast_to(values, (batch,) + values.shape)
    contributions = np.where(mask[None, :, :], coeff * v[:, :, None], v.dtype.type(0))
    flat = mask.ravel()
    np.add.at(out, (slice(None), support.ravel()[flat]),
              contributions.reshape(batch, -1)[:, flat])
    return out


def operators(values, support, mask, n):
    """``(mv, tmv)`` pair; kernels.py:43-49.

    Shared coefficients use a scipy CSR/CSC pair built once: a CSR row sums its
    entries in stored (slot) order and a CSC column in increasing row order,
    the same orders as ``matvec``/``tmatvec``.
    """
    if values.ndim == 2 and support.shape[0]:
        import scipy.sparse as sp

        rows = np.repeat(np.arange(support.shape[0]), support.shape[1])[mask.ravel()]
        cols = support.ravel()[mask.ravel()]
        vals = values.ravel()[mask.ravel()]
        K = sp.csr_matrix((vals, (rows, cols)), shape=(support.shape[0], n))
        KT = sp.csr_matrix((vals, (cols, rows)), shape=(n, support.shape[0]))
        K.sort_indices()
        KT.sort_indices()
        return (lambda x: np.ascontiguousarray((K @ x.T).T).astype(x.dtype, copy=False),
                lambda v: np.ascontiguousarray((KT @ v.T).T).astype(v.dtype, copy=False))
    return (
        lambda x: matvec(values, support, mask, x),
        lambda v: tmatvec(values, support, mask, v, n),
    )


# ---------------------------------------------------------------------------
# step sizes
# ---------------------------------------------------------------------------


def start_vector(n, seed, dtype):
    """Deterministic power-iteration start vector (this build's own generator).

    splitmix64 of ``seed*2^32 + j`` mapped to ``[-1, 1)``.  The reference uses
    ``jax.random.normal(split(PRNGKey(seed), B))`` (kernels.py:54-55), which is
    not reproducible without JAX; any generic start vector gives a valid
    estimate.  The HIP library builds the identical vector
    (purin_amd/csrc/plan.cpp).
    """
    mask64 = (1 << 64) - 1
    out = np.empty(n, dtype=np.float64)
    for j in range(n):
        z = ((seed << 32) + j + 0x9E3779B97F4A7C15) & mask64
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask64
        z = z ^ (z >> 31)
        out[j] = (z >> 11) * (2.0 ** -53) * 2.0 - 1.0
    return out.astype(dtype)


def _sum_in_order(a):
    """Row sums of ``a`` (B, n) added in column order, each addition rounded."""
    acc = np.zeros(a.shape[0], a.dtype)
    for j in range(a.shape[1]):
        acc = acc + a[:, j]
    return acc


def norm_estimate(mv, tmv, batch, n, dtype, iterations=20, seed=42):
    """Power iteration on ``K^T K``; kernels.py:52-65.

    All samples start from the same ``start_vector`` (see its docstring).  The
    dot products add in index order (the HIP library's order; the reference's
    ``jnp.sum`` leaves its reduction order to XLA).
    """
    dtype = np.dtype(dtype)
    x = np.broadcast_to(start_vector(n, seed, dtype), (batch, n)).copy()
    eps = dtype.type(1e-12)
    x = x / (np.sqrt(_sum_in_order(x * x))[:, None] + eps)
    eig = np.zeros(batch, dtype)
    for _ in range(iterations):
        z = tmv(mv(x))
        eig = _sum_in_order(x * z)
        x = z / (np.sqrt(_sum_in_order(z * z))[:, None] + eps)
    return np.sqrt(np.maximum(eig, dtype.type(0))) + eps


def norm_bound(values, support, mask, batch, n, dtype):
    """Sparse bound ``sqrt(max_i sum_j |K_ij| * max_j sum_i |K_ij|)``; kernels.py:213-220."""
    dtype = np.dtype(dtype)
    av = np.abs(values)
    row_sum = matvec(av, support, mask, np.ones((batch, n), dtype))
    col_sum = tmatvec(av, support, mask, np.ones((batch, support.shape[0]), dtype), n)
    rmax = row_sum.max(axis=1, initial=0.0).astype(dtype)
    cmax = col_sum.max(axis=1, initial=0.0).astype(dtype)
    return np.sqrt(rmax * cmax)


def proximal_coefficients(q, c, tau):
    """Fixed diagonal prox ``a*y - d*(K^T dual) + offset``; kernels.py:68-73."""
    step = tau[:, None] if tau.ndim == 1 else tau
    one = q.dtype.type(1)
    inverse = one / (one + step * q)
    dual_weight = step * inverse
    return inverse, dual_weight, -dual_weight * c


def diagonal_step_sizes(q, values, support, mask, safety):
    """Diagonal metrics ``T_j = s/colsum_j``, ``S_i = s/rowsum_i``; kernels.py:76-88."""
    dtype = q.dtype
    av = np.abs(values)
    n = q.shape[1]
    row = matvec(av, support, mask, np.ones_like(q))
    column = tmatvec(av, support, mask, np.ones_like(row), n)
    tiny = dtype.type(1e-12)
    row = np.where(row > 0, np.maximum(row, tiny), dtype.type(1))
    column = np.where(column > 0, np.maximum(column, tiny), dtype.type(1))
    s = dtype.type(safety)
    return s / column, s / row


def step_sizes(q, values, support, mask, *, accelerated, safety, norm_bound_flag,
               diagonal_preconditioning, norm_iterations=20, norm_seed=42):
    """Initial (tau, sigma); kernels.py:209-227."""
    batch, n = q.shape
    dtype = q.dtype
    if diagonal_preconditioning and not accelerated:
        return diagonal_step_sizes(q, values, support, mask, safety)
    mv, tmv = operators(values, support, mask, n)
    if norm_bound_flag:
        norm = norm_bound(values, support, mask, batch, n, dtype)
    else:
        norm = norm_estimate(mv, tmv, batch, n, dtype, norm_iterations, norm_seed)
    L = np.maximum(norm, dtype.type(1e-12))
    s = dtype.type(safety)
    sigma = s / L
    tau = np.where(
        accelerated & (np.min(q, axis=1) > 0), s / L, s / (np.max(q, axis=1) + L)
    ).astype(dtype)
    return tau, sigma


# ---------------------------------------------------------------------------
# iteration
# ---------------------------------------------------------------------------


def clip(x, lower, upper):
    """``jnp.clip`` = ``minimum(maximum(x, lower), upper)``."""
    return np.minimum(np.maximum(x, lower), upper)


def cp_step(state, q, c, rhs, lower, upper, mv, tmv, me, tau, sigma, theta,
            proximal=None, return_pre_clip=False, factored_proximal=False):
    """One CP primal/dual update plus extrapolation; kernels.py:91-150.

    ``factored_proximal`` selects the dense adapter's arithmetic
    ``inverse * ((y - tau K^T d) - tau c)`` (kernels.py:140-142).
    """
    y, dual, ybar = state
    dual_step = sigma[:, None] if sigma.ndim == 1 else sigma
    next_dual = dual + dual_step * (mv(ybar) - rhs)
    next_dual = np.concatenate(
        (next_dual[:, :me], np.maximum(next_dual[:, me:], next_dual.dtype.type(0))), axis=1
    )
    inverse, dual_weight, offset = (
        proximal_coefficients(q, c, tau) if proximal is None else proximal
    )
    if factored_proximal:
        step = tau[:, None] if tau.ndim == 1 else tau
        pre = inverse * ((y - step * tmv(next_dual)) - step * c)
    else:
        pre = inverse * y - dual_weight * tmv(next_dual) + offset
    next_y = clip(pre, lower, upper)
    th = theta[:, None]
    out = (next_y, next_dual, next_y + th * (next_y - y))
    if return_pre_clip:
        return out, pre
    return out


def diagnostics(y, dual, q, c, rhs, lower, upper, mv, tmv, me):
    """Feasibility violation and normalized gap; kernels.py:153-175."""
    dtype = y.dtype
    zero = dtype.type(0)
    residuals = mv(y) - rhs
    eq = np.max(np.abs(residuals[:, :me]), axis=1, initial=0.0).astype(dtype)
    ineq = np.max(np.maximum(residuals[:, me:], zero), axis=1, initial=0.0).astype(dtype)
    bound = np.maximum(
        np.max(np.maximum(lower - y, zero), axis=1, initial=0.0),
        np.max(np.maximum(y - upper, zero), axis=1, initial=0.0),
    ).astype(dtype)
    half = dtype.type(0.5)
    primal = np.sum(half * q * y * y + c * y, axis=1)
    t = c + tmv(dual)
    positive = q > 1e-12
    free = -t / np.where(positive, q, dtype.type(1))
    minimizer = np.where(
        positive, clip(free, lower, upper), np.where(t >= 0.0, lower, upper)
    )
    dual_objective = np.sum(half * q * minimizer**2 + t * minimizer, axis=1) - np.sum(
        rhs * dual, axis=1
    )
    gap = np.maximum(primal - dual_objective, zero) / np.maximum(
        dtype.type(1), np.maximum(np.abs(primal), np.abs(dual_objective))
    )
    return np.maximum(np.maximum(eq, ineq), bound), gap


def stationarity(y, dual, q, c, lower, upper, tmv):
    """``max |y - clip(y - (q y + c + K^T d), lo, hi)|``; kernels.py:272-274."""
    return np.max(np.abs(y - clip(y - (q * y + c + tmv(dual)), lower, upper)), axis=1)


def sparse_cp(q, c, values, rhs, support, mask, me, lower, upper, *,
              accelerated=False, safety=0.95, max_iterations=5000, tolerance=1e-9,
              norm_iterations=20, norm_seed=42, y0=None, dual0=None,
              freeze_converged=False, check_stationarity=False, norm_bound=False,
              diagonal_preconditioning=False, early_stop=True, steps=None, trace=None,
              factored_proximal=False):
    """Batched diagonal-QP CP solve; kernels.py:178-305.

    ``early_stop=False`` is this build's explicit fixed-iteration mode: the
    per-iteration acceptance test never fires (the reference reaches the same
    state with a tolerance too small to be met), so every sample runs exactly
    ``max_iterations`` iterations.  The final diagnostics (kernels.py:291-305)
    still use ``tolerance``.  ``steps`` optionally overrides the initial
    ``(tau, sigma)``.  ``trace``: a list that receives, per iteration, each
    sample's stop-test margin ``max(residual, gap[, stationarity]) / tolerance``
    (test diagnostics: a margin within rounding of 1 marks a sample whose stop
    iteration rounding can move).
    """
    dtype = q.dtype
    batch, n = q.shape
    mv, tmv = operators(values, support, mask, n)
    if steps is None:
        tau, sigma = step_sizes(
            q, values, support, mask, accelerated=accelerated, safety=safety,
            norm_bound_flag=norm_bound, diagonal_preconditioning=diagonal_preconditioning,
            norm_iterations=norm_iterations, norm_seed=norm_seed)
    else:
        tau, sigma = (np.asarray(s, dtype) for s in steps)
    gamma = np.min(q, axis=1)
    y = np.zeros_like(q) if y0 is None else np.array(y0, dtype=dtype)
    dual = np.zeros_like(rhs) if dual0 is None else np.array(dual0, dtype=dtype)
    ybar = y.copy()
    theta = np.ones(batch, dtype)
    done = np.zeros(batch, bool)
    counts = np.zeros(batch, np.int32)
    tolerance = np.asarray(tolerance, dtype=dtype)
    proximal = None if accelerated else proximal_coefficients(q, c, tau)
    iteration = 0
    while iteration < max_iterations and not np.all(done):
        ny, nd, nb = cp_step((y, dual, ybar), q, c, rhs, lower, upper, mv, tmv, me,
                             tau, sigma, theta, proximal=proximal,
                             factored_proximal=factored_proximal)
        active = ~done if freeze_converged else np.ones_like(done)
        if early_stop:
            residual, gap = diagnostics(ny, nd, q, c, rhs, lower, upper, mv, tmv, me)
            finite = (np.all(np.isfinite(ny), axis=1) & np.all(np.isfinite(nd), axis=1)
                      & np.isfinite(gap))
            accepted = finite & (residual <= tolerance) & (gap <= tolerance)
            if check_stationarity:
                stat = stationarity(ny, nd, q, c, lower, upper, tmv)
                accepted = accepted & (stat <= tolerance)
            if trace is not None:
                worst = np.maximum(residual, gap)
                if check_stationarity:
                    worst = np.maximum(worst, stat)
                trace.append(worst / tolerance)
        y = np.where(active[:, None], ny, y)
        dual = np.where(active[:, None], nd, dual)
        ybar = np.where(active[:, None], nb, ybar)
        counts = counts + active.astype(np.int32)
        if early_stop:
            done = done | accepted
        if accelerated:
            tau, sigma, theta = accelerated_update(tau, sigma, gamma)
        iteration += 1
    residual, gap = diagnostics(y, dual, q, c, rhs, lower, upper, mv, tmv, me)
    finite = (np.all(np.isfinite(y), axis=1) & np.all(np.isfinite(dual), axis=1)
              & np.isfinite(gap) & np.isfinite(residual))
    converged = finite & (residual <= tolerance) & (gap <= tolerance)
    if check_stationarity:
        stat = stationarity(y, dual, q, c, lower, upper, tmv)
        converged = converged & (stat <= tolerance)
        residual = np.maximum(residual, stat)
    return CPOutput(y, dual, counts, residual, gap, converged)


def accelerated_update(tau, sigma, gamma):
    """One accelerated step update; kernels.py:279-283.

    ``nu = 1/sqrt(1 + gamma tau)``; returns ``(nu tau, sigma/nu, nu)`` (the next
    tau, sigma and theta), in the dtype of ``tau``.
    """
    tau = np.asarray(tau)
    one = tau.dtype.type(1)
    nt = one / np.sqrt(one + np.asarray(gamma, tau.dtype) * tau)
    return nt * tau, np.asarray(sigma, tau.dtype) / nt, nt


def accelerated_schedule(tau0, sigma0, iterations, dtype, gamma=1.0):
    """Per-iteration ``(tau, sigma, theta)`` of the accelerated update; kernels.py:279-283.

    Row ``k`` holds the scalars iteration ``k`` uses (theta_0 = 1); each row
    follows from the previous by ``accelerated_update``, the update the loop of
    ``sparse_cp`` applies.
    """
    dtype = np.dtype(dtype)
    g = dtype.type(gamma)
    tau = dtype.type(tau0)
    sigma = dtype.type(sigma0)
    theta = dtype.type(1)
    out = np.empty((iterations, 3), dtype)
    for k in range(iterations):
        out[k] = (tau, sigma, theta)
        tau, sigma, theta = accelerated_update(tau, sigma, g)
    return out
