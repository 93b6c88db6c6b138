"""NumPy restatement of PURIN's prepared CP projection (bound presolve path).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows ``solvers/chambolle_pock/bounds.py:170-326`` (singleton-inequality bound
presolve, row scaling, dual recovery, original-unit diagnostics and status) and
its no-bound twin ``solvers/chambolle_pock/solver.py:277-366``.  With no
singleton inequality rows the two coincide (``feasible`` is then vacuously
true), so one function covers both.

Pinned by: the reference's known-answer cases restated in
``tests/test_oracle_projection.py`` (values, multipliers, slacks, status codes)
and by brute-force active-set QP solutions (``oracle/qp.py``).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import NamedTuple

import numpy as np

from oracle import cp as _cp

CONVERGED, MAX_ITERATIONS, LINEAR_SOLVE_FAILURE, NONFINITE = 0, 1, 2, 3


class ProjectionResult(NamedTuple):
    """solvers/types.py:46-57."""

    y: np.ndarray
    multipliers_eq: np.ndarray
    multipliers_ineq: np.ndarray
    slacks: np.ndarray
    status: np.ndarray
    iterations: np.ndarray
    residual_inf_norm: np.ndarray
    finite: np.ndarray
    gradient_eligible: np.ndarray


@dataclass(frozen=True)
class Config:
    """The ChambollePockConfig knobs the path honours; chambolle_pock/config.py:34-48."""

    tolerance: float = 1e-9
    max_iterations: int = 10000
    accelerated: bool = False
    safety: float = 0.95
    norm_iterations: int = 20
    norm_seed: int = 42
    row_scaling: bool = True
    norm_bound: bool = True
    diagonal_preconditioning: bool = False
    early_stop: bool = True
    # linear solver / implicit gradient (solvers/config.py:13-16, 94)
    gmres_tolerance: float = 1e-9
    gmres_atol: float = 0.0
    gmres_restart: int = 30
    gmres_max_iterations: int = 100
    adjoint_tolerance: float = 1e-8


@dataclass
class Canonical:
    """Shared-coefficient canonical rows: ``K[:me] y = rhs[:me]``, ``K[me:] y <= rhs[me:]``.

    ``rows`` lists the (ascending) columns of each row; ``coef`` the matching
    values.  This is the numeric content of ``_numeric_one`` (solver.py:87-138)
    when the coefficients do not depend on parameters.
    """

    n: int
    me: int
    rows: list
    coef: list

    @property
    def mi(self):
        return len(self.rows) - self.me

    def ell(self, dtype):
        support, mask = _cp.layout(self.rows, self.n)
        values = np.zeros(support.shape, dtype=dtype)
        for i, vals in enumerate(self.coef):
            values[i, : len(vals)] = np.asarray(vals, dtype=dtype)
        return support, mask, values

    def dense(self, dtype=np.float64):
        out = np.zeros((len(self.rows), self.n), dtype)
        for i, (cols, vals) in enumerate(zip(self.rows, self.coef)):
            out[i, list(cols)] = vals
        return out


def bound_rows(canon):
    """Singleton inequality rows; bounds.py:320-326."""
    return [canon.me + i for i, row in enumerate(canon.rows[canon.me:]) if len(row) == 1]


class Presolved(NamedTuple):
    support: np.ndarray
    mask: np.ndarray
    values: np.ndarray          # full (M, w) coefficients
    rows: np.ndarray            # kept row indices
    bounds: np.ndarray          # bound row indices
    variables: np.ndarray       # variable of each bound row
    scale: np.ndarray           # (B, m_kept)
    lower: np.ndarray
    upper: np.ndarray
    feasible: np.ndarray
    coefficient: np.ndarray
    threshold: np.ndarray
    kept_values: np.ndarray     # scaled kept coefficients (B, m, w)
    kept_rhs: np.ndarray        # scaled kept rhs (B, m)
    tolerance: np.ndarray


def presolve(canon, rhs, cfg, dtype, values=None):
    """Bounds, feasibility and row scaling; bounds.py:192-236.

    ``values``: per-sample coefficients ``(B, M, w)`` on ``canon``'s ELL support
    (the reference's ``jax.vmap(_numeric_one)(theta)`` values, bounds.py:192);
    ``None`` uses ``canon``'s shared coefficients.
    """
    dtype = np.dtype(dtype)
    support, mask, shared = canon.ell(dtype)
    values = shared if values is None else np.where(mask[None], np.asarray(values, dtype), 0)
    batch = rhs.shape[0]
    bidx = np.asarray(bound_rows(canon), dtype=np.int64)
    bset = set(bidx.tolist())
    rows = np.asarray([r for r in range(len(canon.rows)) if r not in bset], dtype=np.int64)
    variables = support[bidx, 0] if len(bidx) else np.zeros(0, np.int32)
    vals_b = values if values.ndim == 3 else np.broadcast_to(values, (batch,) + values.shape)
    coefficient = vals_b[:, bidx, 0] if len(bidx) else np.zeros((batch, 0), dtype)
    threshold = rhs[:, bidx] / np.where(coefficient != 0, coefficient, dtype.type(1))
    lower = np.full((batch, canon.n), -np.inf, dtype)
    upper = np.full((batch, canon.n), np.inf, dtype)
    for k in range(len(bidx)):
        j = variables[k]
        lower[:, j] = np.maximum(lower[:, j], np.where(coefficient[:, k] < 0, threshold[:, k], -np.inf))
        upper[:, j] = np.minimum(upper[:, j], np.where(coefficient[:, k] > 0, threshold[:, k], np.inf))
    feasible = np.all(lower <= upper, axis=1) & np.all(
        (coefficient != 0) | (rhs[:, bidx] >= 0), axis=1)
    kept = vals_b[:, rows]
    scale = np.ones((batch, len(rows)), dtype)
    if cfg.row_scaling and len(rows):
        norms = np.sqrt(np.sum(kept ** 2, axis=2))
        scale = np.where(norms > 0, dtype.type(1) / np.maximum(norms, dtype.type(1e-30)),
                         dtype.type(1)).astype(dtype)
    tolerance = (dtype.type(cfg.tolerance)
                 * np.minimum(dtype.type(1), np.min(scale, axis=1, initial=1.0))).astype(dtype)
    return Presolved(support, mask, values, rows, bidx, variables, scale, lower, upper,
                     feasible, coefficient, threshold, kept * scale[:, :, None],
                     rhs[:, rows] * scale, tolerance)


def solve(canon, target, rhs, cfg, *, dtype=np.float64, multipliers_eq=None,
          multipliers_ineq=None, return_internal=False, values=None, trace=None):
    """``BoundProjection.solve`` (bounds.py:170-317).

    ``rhs`` is ``-[h(theta,0); g(theta,0)]`` for all ``me+mi`` rows (solver.py:132-137);
    ``values`` optional per-sample coefficients ``(B, M, w)`` (see ``presolve``).
    """
    dtype = np.dtype(dtype)
    target = np.asarray(target, dtype)
    rhs = np.asarray(rhs, dtype)
    batch, n = target.shape
    me = canon.me
    pre = presolve(canon, rhs, cfg, dtype, values)
    eq = np.zeros((batch, me), dtype) if multipliers_eq is None else np.asarray(multipliers_eq, dtype)
    iq = (np.zeros((batch, canon.mi), dtype) if multipliers_ineq is None
          else np.asarray(multipliers_ineq, dtype))
    initial = np.concatenate((eq, iq), axis=1)[:, pre.rows] / pre.scale
    ksup, kmask = pre.support[pre.rows], pre.mask[pre.rows]
    out = _cp.sparse_cp(
        np.ones_like(target), -target, pre.kept_values, pre.kept_rhs, ksup, kmask, me,
        pre.lower, pre.upper, accelerated=cfg.accelerated, safety=cfg.safety,
        max_iterations=cfg.max_iterations, tolerance=pre.tolerance,
        norm_iterations=cfg.norm_iterations, norm_seed=cfg.norm_seed, y0=target,
        dual0=initial, freeze_converged=True, check_stationarity=True,
        norm_bound=cfg.norm_bound, diagonal_preconditioning=cfg.diagonal_preconditioning,
        early_stop=cfg.early_stop, trace=trace)
    out = out._replace(converged=out.converged & pre.feasible)
    result = recover(canon, pre, out, target, rhs, cfg)
    if return_internal:
        return result, out, pre
    return result


def recover(canon, pre, out, target, rhs, cfg):
    """Dual placement, bound-multiplier recovery, residual and status; bounds.py:247-317."""
    dtype = target.dtype
    zero = dtype.type(0)
    me = canon.me
    n = canon.n
    dual = np.zeros_like(rhs)
    dual[:, pre.rows] = out.dual * pre.scale
    mv, tmv = _cp.operators(pre.values, pre.support, pre.mask, n)
    if len(pre.bounds):
        base = out.y - target + tmv(dual)
        var = pre.variables
        lo_v, hi_v, y_v = pre.lower[:, var], pre.upper[:, var], out.y[:, var]
        is_lower = (pre.coefficient < 0) & (pre.threshold == lo_v) & (y_v == lo_v)
        is_upper = (pre.coefficient > 0) & (pre.threshold == hi_v) & (y_v == hi_v)
        lower_count = np.zeros_like(target)
        upper_count = np.zeros_like(target)
        np.add.at(lower_count, (slice(None), var), is_lower.astype(dtype))
        np.add.at(upper_count, (slice(None), var), is_upper.astype(dtype))
        normal = base[:, var]
        one = dtype.type(1)
        bound_dual = np.where(is_lower, np.maximum(normal, zero)
                              / np.maximum(lower_count[:, var], one), zero)
        bound_dual = bound_dual + np.where(is_upper, np.maximum(-normal, zero)
                                           / np.maximum(upper_count[:, var], one), zero)
        bound_dual = bound_dual / np.where(pre.coefficient != 0, np.abs(pre.coefficient), one)
        dual[:, pre.bounds] = bound_dual
    r = mv(out.y) - rhs
    eq_res = np.max(np.abs(r[:, :me]), axis=1, initial=0.0).astype(dtype)
    iq_res = np.max(np.maximum(r[:, me:], zero), axis=1, initial=0.0).astype(dtype)
    stationarity = np.max(np.abs(out.y - target + tmv(dual)), axis=1)
    residual = np.maximum(np.maximum(eq_res, iq_res), stationarity)
    finite = (np.all(np.isfinite(out.y), axis=1) & np.all(np.isfinite(dual), axis=1)
              & np.isfinite(residual) & np.isfinite(out.gap))
    converged = finite & out.converged & (residual <= dtype.type(cfg.tolerance))
    status = np.where(converged, CONVERGED,
                      np.where(finite, MAX_ITERATIONS, NONFINITE)).astype(np.int32)
    return ProjectionResult(out.y, dual[:, :me], dual[:, me:], np.maximum(-r[:, me:], zero),
                            status, out.iterations, residual, finite, converged)


def row_scaling_pullback(kept, mask, rhs, g_scaled, g_rhs_scaled, row_scaling):
    """Pull gradients w.r.t. the scaled rows ``(s K, s r)`` back to ``(K, r)``.

    ``s_i = 1/max(||K_i||, 1e-30)`` for a nonzero row, else 1, and 1 without
    row scaling (bounds.py:210-214, 228-230).  Returns
    ``g_K = s g~_K - s^3 K (sum_j g~_K K + g~_r r)`` (the second term when row
    scaling is on and ``||K_i|| > 1e-30``; the reference's graph gives NaN for an
    all-zero row through ``sqrt'(0)``, this restatement takes the limit 0) and
    ``g_r = s g~_r``.
    """
    kept = np.where(mask[None], kept, 0)
    norms = np.sqrt(np.sum(kept ** 2, axis=2))
    one = kept.dtype.type(1)
    if row_scaling:
        scale = np.where(norms > 0, one / np.maximum(norms, kept.dtype.type(1e-30)), one)
    else:
        scale = np.ones_like(norms)
    s = scale[:, :, None]
    g_scale = np.sum(np.where(mask[None], g_scaled * kept, 0), axis=2) + g_rhs_scaled * rhs
    chain = (norms > 1e-30) if row_scaling else np.zeros_like(norms, bool)
    g_kept = g_scaled * s - np.where(chain[:, :, None], s ** 3 * g_scale[:, :, None] * kept, 0)
    return np.where(mask[None], g_kept, 0), g_rhs_scaled * scale


def vjp(canon, target, rhs, cfg, cot_y, *, dtype=np.float64, values=None,
        return_values=False, state=None):
    """Forward solve plus implicit VJP w.r.t. ``target``, all ``rhs`` rows and,
    with ``return_values``, the coefficients.

    The adjoint is bounds.py:80-165 (``oracle.adjoint.adjoint``); the chain rule
    through the presolve follows the JAX graph of bounds.py:193-239:
    * kept rows: ``K~ = s K``, ``r~ = s r`` with ``s = 1/max(||K_i||, 1e-30)``
      (1 for a zero row or without row scaling), so ``g_r = g_r~ s`` and
      ``g_K = s g_K~ - s^3 K (sum_j g_K~_ij K_ij + g_r~_i r_i)`` (the second
      term when row scaling is on and ``||K_i|| > 1e-30``; the reference's graph
      gives NaN for an all-zero row there, through ``sqrt'(0)``, and this
      restatement takes the limit 0);
    * bound rows: ``threshold = rhs / c`` reaches ``lower``/``upper`` through
      scatter max/min; a bound row's ``g_threshold`` is its variable's
      ``g_lower``/``g_upper`` when it attains the bound (ties split evenly:
      this build's choice, unpinned by the reference), ``g_rhs = g_thr / c``
      and ``g_c = -g_thr rhs / c^2``.
    Returns ``(result, g_target, g_rhs, adjoint_result)`` and, with
    ``return_values``, ``g_values`` ``(B, M, w)`` on ``canon``'s ELL support
    after them.  ``state = (y, scaled kept dual)`` linearises at that state
    instead of this oracle's own solution (the forward result is still the
    oracle's).
    """
    from oracle import adjoint as _adj

    dtype = np.dtype(dtype)
    target = np.asarray(target, dtype)
    rhs = np.asarray(rhs, dtype)
    result, out, pre = solve(canon, target, rhs, cfg, dtype=dtype, return_internal=True,
                             values=values)
    ksup, kmask = pre.support[pre.rows], pre.mask[pre.rows]
    y_lin, d_lin = (out.y, out.dual) if state is None else (np.asarray(state[0], dtype),
                                                            np.asarray(state[1], dtype))
    adj = _adj.adjoint(pre.kept_values, ksup, kmask, canon.me, y_lin, d_lin,
                       out.converged, target, pre.kept_rhs, pre.lower, pre.upper,
                       np.asarray(cot_y, dtype), cfg)
    batch = target.shape[0]
    g_rhs = np.zeros_like(rhs)
    vals_b = (pre.values if pre.values.ndim == 3
              else np.broadcast_to(pre.values, (batch,) + pre.values.shape))
    g_values = np.zeros(vals_b.shape, dtype)
    if len(pre.rows):
        g_kept, g_rhs[:, pre.rows] = row_scaling_pullback(
            vals_b[:, pre.rows], kmask, rhs[:, pre.rows], adj.g_values, adj.g_rhs,
            cfg.row_scaling)
        g_values[:, pre.rows] = g_kept
    for k, r in enumerate(pre.bounds):
        j = pre.variables[k]
        coef = pre.coefficient[:, k]
        lo_hit = (coef < 0) & (pre.threshold[:, k] == pre.lower[:, j])
        hi_hit = (coef > 0) & (pre.threshold[:, k] == pre.upper[:, j])
        same = pre.variables == j
        n_lo = np.sum((pre.coefficient[:, same] < 0)
                      & (pre.threshold[:, same] == pre.lower[:, j][:, None]), axis=1)
        n_hi = np.sum((pre.coefficient[:, same] > 0)
                      & (pre.threshold[:, same] == pre.upper[:, j][:, None]), axis=1)
        g_thr = (np.where(lo_hit, adj.g_lower[:, j] / np.maximum(n_lo, 1), 0)
                 + np.where(hi_hit, adj.g_upper[:, j] / np.maximum(n_hi, 1), 0))
        safe = np.where(coef != 0, coef, 1)
        g_rhs[:, r] = np.where(coef != 0, g_thr / safe, g_thr)
        g_values[:, r, 0] = np.where(coef != 0, -g_thr * rhs[:, r] / safe ** 2, 0)
    if return_values:
        return result, adj.g_target, g_rhs, adj, g_values
    return result, adj.g_target, g_rhs, adj
