"""NumPy restatement of PURIN's general diagonal-QP layer.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows ``src/purin/solvers/diagonal_qp.py``: ``PreparedDiagonalQP.solve``
(222-319: stop-gradient row scaling, scaled tolerance, ``sparse_cp`` with a
general positive diagonal ``q``, validity ``q > 0`` and ``lower <= upper``,
original-unit residual with the clip stationarity, status, slacks) and the
custom_vjp ``bwd`` (131-219: steps from the norm bound or the power iteration
with ``tau = s/(max q + L)``, or the diagonal steps; GMRES on
``(I - J^T) lambda = [cot_y, cot_dual, 0] * converged``; the pullback w.r.t.
``q, c, values, rhs, lower, upper``).

Pinned by: the reference's known answer (tests/test_diagonal_qp.py:13-48:
``q = [2, 4]``, ``c = [-2, -4]``, ``u + v = 1`` gives ``[1/3, 2/3]`` and the
closed-form ``dy/dc``), exact QP solutions by active-set enumeration
(``oracle/qp.py`` after the substitution ``z = sqrt(q) y``) and central
differences of those exact solutions in every input
(tests/test_oracle_diagonal_qp.py).
"""

from __future__ import annotations

from typing import NamedTuple

import numpy as np

from oracle import adjoint as _adj
from oracle import cp as _cp
from oracle.projection import CONVERGED, MAX_ITERATIONS, NONFINITE, ProjectionResult


class QPData(NamedTuple):
    """diagonal_qp.py:26-34 (values on the ELL support, (B, m, w))."""

    q: np.ndarray
    c: np.ndarray
    values: np.ndarray
    rhs: np.ndarray
    lower: np.ndarray
    upper: np.ndarray


def _scale(data, mask, cfg):
    """Row scales 1/||K_i|| (1 for a zero row, all 1 without row scaling); diagonal_qp.py:250-256."""
    dtype = data.values.dtype
    one = dtype.type(1)
    if not cfg.row_scaling:
        return np.ones_like(data.rhs)
    norms = np.sqrt(np.sum(np.where(mask[None], data.values ** 2, 0), axis=2))
    return np.where(norms > 0, one / np.maximum(norms, dtype.type(1e-30)), one).astype(dtype)


def solve(support, mask, me, data, cfg, *, y0=None, dual0=None, trace=None,
          return_internal=False):
    """``PreparedDiagonalQP.solve``; diagonal_qp.py:222-319."""
    dtype = data.q.dtype
    zero = dtype.type(0)
    batch, n = data.q.shape
    values = np.where(mask[None], data.values, 0).astype(dtype)
    data = data._replace(values=values)
    scale = _scale(data, mask, cfg)
    scaled_values = values * scale[:, :, None]
    scaled_rhs = data.rhs * scale
    tolerance = (dtype.type(cfg.tolerance)
                 * np.minimum(dtype.type(1), np.min(scale, axis=1, initial=1.0))).astype(dtype)
    y_init = np.zeros((batch, n), dtype) if y0 is None else np.asarray(y0, dtype)
    d_init = (np.zeros_like(data.rhs) if dual0 is None else np.asarray(dual0, dtype)) / scale
    out = _cp.sparse_cp(
        data.q, data.c, scaled_values, scaled_rhs, support, mask, me, data.lower, data.upper,
        accelerated=cfg.accelerated, safety=cfg.safety, max_iterations=cfg.max_iterations,
        tolerance=tolerance, norm_iterations=cfg.norm_iterations, norm_seed=cfg.norm_seed,
        y0=y_init, dual0=d_init, freeze_converged=True, check_stationarity=True,
        norm_bound=cfg.norm_bound, diagonal_preconditioning=cfg.diagonal_preconditioning,
        early_stop=cfg.early_stop, trace=trace)
    valid = np.all(data.q > 0, axis=1) & np.all(data.lower <= data.upper, axis=1)
    out = out._replace(converged=out.converged & valid)
    dual = out.dual * scale
    mv, tmv = _cp.operators(values, support, mask, n)
    r = mv(out.y) - data.rhs
    eq = np.max(np.abs(r[:, :me]), axis=1, initial=0.0).astype(dtype)
    iq = np.max(np.maximum(r[:, me:], zero), axis=1, initial=0.0).astype(dtype)
    stat = np.max(np.abs(out.y - _cp.clip(out.y - (data.q * out.y + data.c + tmv(dual)),
                                          data.lower, data.upper)), axis=1)
    residual = np.maximum(np.maximum(eq, iq), stat)
    converged = out.converged & (residual <= dtype.type(cfg.tolerance))
    finite = (np.all(np.isfinite(out.y), axis=1) & np.all(np.isfinite(dual), axis=1)
              & np.isfinite(residual))
    status = np.where(converged, CONVERGED,
                      np.where(finite, MAX_ITERATIONS, NONFINITE)).astype(np.int32)
    slacks = np.maximum(-r[:, me:], zero)
    result = ProjectionResult(out.y, dual[:, :me], dual[:, me:], slacks, status, out.iterations,
                              residual, finite, converged)
    if return_internal:
        return result, out, (scale, scaled_values, scaled_rhs)
    return result


class QPGradients(NamedTuple):
    q: np.ndarray
    c: np.ndarray
    values: np.ndarray
    rhs: np.ndarray
    lower: np.ndarray
    upper: np.ndarray


def adjoint_steps(support, mask, data, scaled_values, cfg):
    """The backward's steps; diagonal_qp.py:137-160."""
    dtype = data.q.dtype
    batch, n = data.q.shape
    if cfg.diagonal_preconditioning and not cfg.accelerated:
        return _cp.diagonal_step_sizes(data.q, scaled_values, support, mask, cfg.safety)
    if cfg.norm_bound:
        L = _cp.norm_bound(scaled_values, support, mask, batch, n, dtype)
    else:
        mv, tmv = _cp.operators(scaled_values, support, mask, n)
        L = _cp.norm_estimate(mv, tmv, batch, n, dtype, cfg.norm_iterations, cfg.norm_seed)
    L = np.maximum(L, dtype.type(1e-12))
    s = dtype.type(cfg.safety)
    return (s / (np.max(data.q, axis=1) + L)).astype(dtype), (s / L).astype(dtype)


def vjp(support, mask, me, data, cfg, cot_y, cot_dual=None, *, state=None):
    """Solve, then the implicit VJP; diagonal_qp.py:131-219 and the stop-gradient
    row scaling of 250-274 (gradients w.r.t. the scaled values and rhs are
    multiplied by the scale; the returned multipliers are ``dual * scale``, so
    the dual cotangent enters as ``cot_dual * scale``).  ``state = (y, scaled
    dual)`` linearises there instead of at this oracle's own solution.
    Returns ``(result, QPGradients, adjoint_result)``.
    """
    dtype = data.q.dtype
    result, out, (scale, scaled_values, scaled_rhs) = solve(support, mask, me, data, cfg,
                                                            return_internal=True)
    y, dual = (out.y, out.dual) if state is None else (np.asarray(state[0], dtype),
                                                       np.asarray(state[1], dtype))
    steps = adjoint_steps(support, mask, data, scaled_values, cfg)
    cd = None if cot_dual is None else np.asarray(cot_dual, dtype) * scale
    adj = _adj.adjoint(scaled_values, support, mask, me, y, dual, out.converged, None,
                       scaled_rhs, data.lower, data.upper, np.asarray(cot_y, dtype), cfg,
                       steps=steps, q=data.q, c=data.c, cot_dual=cd)
    grads = QPGradients(adj.g_q, -adj.g_target, np.where(mask[None], adj.g_values, 0)
                        * scale[:, :, None], adj.g_rhs * scale, adj.g_lower, adj.g_upper)
    return result, grads, adj


def dense_qp_data(q, c, A, b, C, d, lower, upper):
    """diagonal_qp.py:322-349: dense rows over all n variables, broadcast to the batch.

    Returns ``(rows, me, QPData)`` with ``rows`` the (all-column) supports.
    """
    q = np.asarray(q, np.float64)
    c = np.asarray(c, np.float64)
    if q.ndim != 2 or q.shape != c.shape:
        raise ValueError("q and c must be matching batched matrices")
    batch, n = q.shape
    A = np.broadcast_to(np.asarray(A, np.float64), (batch,) + np.shape(A)[-2:])
    C = np.broadcast_to(np.asarray(C, np.float64), (batch,) + np.shape(C)[-2:])
    rows = [list(range(n))] * (A.shape[1] + C.shape[1])
    values = np.concatenate((A, C), axis=1)
    rhs = np.concatenate((np.broadcast_to(b, (batch, A.shape[1])),
                          np.broadcast_to(d, (batch, C.shape[1]))), axis=1)
    return rows, A.shape[1], QPData(q, c, values, rhs, np.broadcast_to(lower, q.shape).copy(),
                                    np.broadcast_to(upper, q.shape).copy())
