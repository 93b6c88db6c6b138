"""NumPy restatement of the CP implicit-differentiation adjoint.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

* ``linearize``/``pullback``: the VJP of one ``cp_step`` (theta = 1, fixed-step
  prox) at the converged state, written in mask form.  ``jax.vjp`` of
  ``step`` in solvers/chambolle_pock/bounds.py:109-130 computes the same map;
  ties of ``maximum``/``clip`` take JAX's balanced 0.5 rule.
  Pinned by: central finite differences of ``oracle.cp.cp_step`` (linear map,
  checked to 1e-7) in tests/test_oracle_adjoint.py.
* ``batched_restarted_gmres``: solvers/primal_dual_interior_point/operators.py:792-1125
  (two-pass classical Gram--Schmidt over the restart prefix, Givens rotations,
  per-sample active masks, back substitution, candidate acceptance).
  Pinned by: ``numpy.linalg.solve`` on small dense systems.
* ``adjoint``: bounds.py:80-165.  Pinned by: the closed-form active-set
  derivative of the exact QP (``oracle/qp.py``) and the reference's
  known-answer gradients (tests/test_oracle_adjoint.py).
"""

from __future__ import annotations

from typing import NamedTuple

import numpy as np

from oracle import cp as _cp


def _max_grads(x, y):
    """d max(x, y)/dx and /dy with JAX's balanced tie rule (0.5 each)."""
    ans = np.maximum(x, y)
    ex, ey = x == ans, y == ans
    dx = np.where(ex, np.where(ey, 0.5, 1.0), 0.0)
    dy = np.where(ey, np.where(ex, 0.5, 1.0), 0.0)
    return ans, dx, dy


def _min_grads(x, y):
    ans = np.minimum(x, y)
    ex, ey = x == ans, y == ans
    dx = np.where(ex, np.where(ey, 0.5, 1.0), 0.0)
    dy = np.where(ey, np.where(ex, 0.5, 1.0), 0.0)
    return ans, dx, dy


class Linearization(NamedTuple):
    values: np.ndarray     # scaled kept coefficients (m, w) or (B, m, w)
    support: np.ndarray
    mask: np.ndarray
    me: int
    n: int
    a: np.ndarray          # (B, 1) prox inverse, or (B, n) for diagonal steps
    delta: np.ndarray      # (B, 1) prox dual weight, or (B, n)
    sigma: np.ndarray      # (B, 1), or (B, m) for diagonal steps
    D: np.ndarray          # dual projection derivative (B, m)
    C: np.ndarray          # clip derivative w.r.t. its argument (B, n)
    Clo: np.ndarray        # clip derivative w.r.t. lower (B, n)
    Chi: np.ndarray        # clip derivative w.r.t. upper (B, n)
    ybar: np.ndarray       # linearization point ybar (= y)
    dplus: np.ndarray      # dual after the step at the linearization point
    q_grad: np.ndarray = None  # (B, n) -tau a s: d(pre-clip s)/dq (general q only)


def linearize(values, support, mask, me, y, dual, target, rhs, lower, upper, tau, sigma,
              q=None, c=None, factored_proximal=False):
    """Masks of ``cp_step`` at ``z = (y, dual, y)`` with theta = 1 (bounds.py:109-128).

    ``tau``/``sigma`` are per sample ``(B,)`` or, with diagonal preconditioning,
    per variable ``(B, n)`` and per row ``(B, m)`` (bounds.py:83-86).  ``q``,
    ``c``: a general diagonal objective (diagonal_qp.py:163-182); default
    ``q = 1``, ``c = -target``.
    """
    dtype = y.dtype
    n = y.shape[1]
    mv, tmv = _cp.operators(values, support, mask, n)
    sig = sigma[:, None] if np.ndim(sigma) == 1 else sigma
    p = dual + sig * (mv(y) - rhs)
    _, dpi, _ = _max_grads(p[:, me:], dtype.type(0))
    D = np.concatenate((np.ones_like(p[:, :me]), dpi.astype(dtype)), axis=1)
    dplus = np.concatenate((p[:, :me], np.maximum(p[:, me:], dtype.type(0))), axis=1)
    general = q is not None
    q = np.ones_like(y) if q is None else np.asarray(q, dtype)
    c = -target if c is None else np.asarray(c, dtype)
    a, delta, offset = _cp.proximal_coefficients(q, c, tau)
    if factored_proximal:  # the dense adapter's arithmetic (kernels.py:140-142)
        step = tau[:, None] if np.ndim(tau) == 1 else tau
        s = a * ((y - step * tmv(dplus)) - step * c)
    else:
        s = a * y - delta * tmv(dplus) + offset
    # d s / d q with a = 1/(1 + tau q), delta = tau a: -tau a s
    q_grad = -(np.broadcast_to(tau[:, None] if np.ndim(tau) == 1 else tau, s.shape) * a * s) \
        if general else None
    m1, ds, dlo = _max_grads(s, lower)
    _, dm1, dhi = _min_grads(m1, upper)
    C = (dm1 * ds).astype(dtype)
    Clo = (dm1 * dlo).astype(dtype)
    Chi = dhi.astype(dtype)
    if np.ndim(tau) == 1 and not general:
        a, delta = a[:, :1], delta[:, :1]  # q = 1: one prox coefficient per sample
    return Linearization(values, support, mask, me, n, a, delta, sig, D, C, Clo, Chi, y.copy(),
                         dplus, q_grad)


class Pullback(NamedTuple):
    gy: np.ndarray
    gd: np.ndarray
    gbar: np.ndarray
    g_values: np.ndarray
    g_rhs: np.ndarray
    g_target: np.ndarray
    g_lower: np.ndarray
    g_upper: np.ndarray
    g_q: np.ndarray = None  # general q only: -tau a u s


def pullback(lin, gy, gd, gb):
    """Transpose Jacobian of the CP step applied to output cotangents.

    With ``G = gy + 2 gb`` (ybar+ = 2 y+ - y), ``u = C*G``,
    ``w = D*(gd - delta K u)``:  state cotangents ``(a u - gb, w, sigma K^T w)``,
    ``g_rhs = -sigma w``, ``g_target = delta u``, ``g_lower = Clo*G``,
    ``g_upper = Chi*G``, ``g_values_ij = sigma w_i ybar_j - delta d+_i u_j``.
    """
    mv, tmv = _cp.operators(lin.values, lin.support, lin.mask, lin.n)
    G = gy + 2 * gb
    u = lin.C * G
    diagonal = lin.delta.shape[1] > 1 or lin.sigma.shape[1] > 1
    if diagonal:
        # per-variable delta and per-row sigma: delta K u -> K (delta u) and
        # sigma K^T w -> K^T (sigma w)
        w = lin.D * (gd - mv(lin.delta * u))
        gz_b = tmv(lin.sigma * w)
    else:
        w = lin.D * (gd - lin.delta * mv(u))
        gz_b = lin.sigma * tmv(w)
    gz_y = lin.a * u - gb
    gz_d = w
    ybar_g = lin.ybar[:, lin.support]
    u_g = u[:, lin.support]
    delta_g = (np.broadcast_to(lin.delta, u.shape)[:, lin.support] if diagonal
               else lin.delta[:, :, None])
    g_values = np.where(lin.mask[None], lin.sigma[:, :, None] * w[:, :, None] * ybar_g
                        - delta_g * lin.dplus[:, :, None] * u_g, 0)
    return Pullback(gz_y, gz_d, gz_b, g_values, -lin.sigma * w, lin.delta * u,
                    lin.Clo * G, lin.Chi * G, None if lin.q_grad is None else lin.q_grad * u)


def batched_restarted_gmres(matvec, rhs, *, tolerance, absolute_tolerance, restart,
                            max_iterations):
    """Restarted batched GMRES; primal_dual_interior_point/operators.py:792-1125.

    Identity preconditioner, ``arnoldi_prefix_block = 0`` (the CGS2 dot
    products run over the zero-padded restart prefix, which is algebraically
    the active prefix), no initial solution.
    Returns ``(x, info, residual_inf, row_iterations)``.
    """
    batch, width = rhs.shape
    dtype = rhs.dtype
    restart = int(min(restart, max_iterations, width))
    eps = dtype.type(1e-30)
    brk = dtype.type(1e-14)
    rhs_scale = np.max(np.abs(rhs), axis=1, initial=0.0).astype(dtype)
    threshold = np.maximum(dtype.type(absolute_tolerance), dtype.type(tolerance) * rhs_scale)

    def norm(v):
        return np.sqrt(np.sum(v * v, axis=1))

    x = np.zeros_like(rhs)
    residual_inf = np.max(np.abs(rhs - matvec(x)), axis=1, initial=0.0).astype(dtype)
    completed = 0
    row_iterations = np.zeros(batch, np.int32)
    while completed < max_iterations and np.any(residual_inf > threshold):
        cycle_limit = min(restart, max_iterations - completed)
        residual = rhs - matvec(x)
        beta = norm(residual)
        safe_beta = np.maximum(beta, eps)
        cycle_active = residual_inf > threshold
        basis = np.zeros((batch, restart + 1, width), dtype)
        basis[:, 0] = residual / safe_beta[:, None]
        precond = np.zeros((batch, restart, width), dtype)
        hess = np.zeros((batch, restart + 1, restart), dtype)
        cos = np.zeros((batch, restart), dtype)
        sin = np.zeros((batch, restart), dtype)
        g = np.zeros((batch, restart + 1), dtype)
        g[:, 0] = beta
        row_steps = np.zeros(batch, np.int32)
        active = cycle_active.copy()
        it = 0
        while it < cycle_limit and np.any(active):
            vector = basis[:, it]
            precond[:, it] = np.where(active[:, None], vector, precond[:, it])
            image = matvec(vector)
            prefix = basis[:, :restart]
            coeff = np.einsum("bid,bd->bi", prefix, image)
            image = image - np.einsum("bi,bid->bd", coeff, prefix)
            corr = np.einsum("bid,bd->bi", prefix, image)
            coeff = coeff + corr
            image = image - np.einsum("bi,bid->bd", corr, prefix)
            next_norm = norm(image)
            safe_norm = np.maximum(next_norm, eps)
            next_vector = image / safe_norm[:, None]
            basis[:, it + 1] = np.where(active[:, None], next_vector, basis[:, it + 1])
            column = np.zeros((batch, restart + 1), dtype)
            column[:, :restart] = coeff
            column[:, it + 1] = next_norm
            for ri in range(restart):
                if ri >= it:
                    break
                first = column[:, ri].copy()
                second = column[:, ri + 1].copy()
                column[:, ri] = cos[:, ri] * first + sin[:, ri] * second
                column[:, ri + 1] = -sin[:, ri] * first + cos[:, ri] * second
            diag = column[:, it]
            sub = column[:, it + 1]
            rnorm = np.hypot(diag, sub)
            safe_r = np.maximum(rnorm, eps)
            nc = np.where(rnorm > eps, diag / safe_r, dtype.type(1))
            ns = np.where(rnorm > eps, sub / safe_r, dtype.type(0))
            cos[:, it] = np.where(active, nc, cos[:, it])
            sin[:, it] = np.where(active, ns, sin[:, it])
            column[:, it] = rnorm
            column[:, it + 1] = 0
            hess[:, :, it] = np.where(active[:, None], column, hess[:, :, it])
            pc, pn = g[:, it].copy(), g[:, it + 1].copy()
            rc = nc * pc + ns * pn
            rn = -ns * pc + nc * pn
            g[:, it] = np.where(active, rc, pc)
            g[:, it + 1] = np.where(active, rn, pn)
            row_steps = np.where(active, it + 1, row_steps)
            est = np.abs(rn)
            finite = np.isfinite(est) & np.isfinite(rnorm) & np.all(np.isfinite(next_vector), axis=1)
            happy = next_norm <= brk
            active = active & finite & ~happy & (est > threshold)
            it += 1
        # back substitution (operators.py:902-917)
        R = hess[:, :restart, :]
        coeffs = np.zeros((batch, restart), dtype)
        for row in range(restart - 1, -1, -1):
            trailing = np.sum(R[:, row, :] * coeffs, axis=1)
            num = g[:, row] - trailing
            d = R[:, row, row]
            safe = np.where(np.abs(d) > eps, d, dtype.type(1))
            coeffs[:, row] = np.where(row < row_steps, num / safe, dtype.type(0))
        correction = np.einsum("bi,bid->bd", coeffs, precond)
        candidate = x + correction
        cand_norm = np.max(np.abs(rhs - matvec(candidate)), axis=1, initial=0.0).astype(dtype)
        x = np.where(cycle_active[:, None], candidate, x)
        residual_inf = np.where(cycle_active, cand_norm, residual_inf)
        completed += it
        row_iterations = row_iterations + row_steps
    finite = np.all(np.isfinite(x), axis=1) & np.isfinite(residual_inf)
    info = np.where(~finite, 2, np.where(residual_inf <= threshold, 0, 1)).astype(np.int32)
    return x, info, residual_inf, row_iterations


class AdjointResult(NamedTuple):
    g_values: np.ndarray
    g_rhs: np.ndarray       # w.r.t. the scaled kept rhs
    g_target: np.ndarray
    g_lower: np.ndarray
    g_upper: np.ndarray
    valid: np.ndarray
    info: np.ndarray
    residual: np.ndarray
    lam: np.ndarray
    tau: np.ndarray
    sigma: np.ndarray
    g_q: np.ndarray = None
    iterations: np.ndarray = None  # per-sample Arnoldi steps (operators.py:1092-1097)


def adjoint_steps(values, support, mask, n, batch, dtype, cfg):
    """Adjoint step sizes from the power-iteration norm estimate; bounds.py:83-101."""
    dtype = np.dtype(dtype)
    mv, tmv = _cp.operators(values, support, mask, n)
    if cfg.diagonal_preconditioning and not cfg.accelerated:
        return _cp.diagonal_step_sizes(np.ones((batch, n), dtype), values, support, mask,
                                       cfg.safety)
    L = np.maximum(_cp.norm_estimate(mv, tmv, batch, n, dtype, cfg.norm_iterations,
                                     cfg.norm_seed), dtype.type(1e-12))
    s = dtype.type(cfg.safety)
    return s / (dtype.type(1) + L), s / L


def adjoint(values, support, mask, me, y, dual, converged, target, rhs, lower, upper,
            cot_y, cfg, steps=None, q=None, c=None, cot_dual=None):
    """Custom-VJP backward of the CP solve; bounds.py:80-165 (solver.py:186-272).

    With ``q``, ``c`` (and optionally ``cot_dual``, the dual's cotangent) it is
    the general diagonal QP's backward, diagonal_qp.py:131-219; the caller
    then passes its ``steps``.  ``g_target`` is ``delta u``; the QP's
    ``g_c`` is its negative.
    """
    dtype = y.dtype
    batch, n = y.shape
    m = dual.shape[1]
    tau, sigma = adjoint_steps(values, support, mask, n, batch, dtype, cfg) if steps is None else steps
    lin = linearize(values, support, mask, me, y, dual, target, rhs, lower, upper, tau, sigma,
                    q=q, c=c)

    def operator(v):
        pb = pullback(lin, v[:, :n], v[:, n:n + m], v[:, n + m:])
        return v - np.concatenate((pb.gy, pb.gd, pb.gbar), axis=1)

    gd0 = np.zeros_like(dual) if cot_dual is None else np.asarray(cot_dual, dtype)
    g = np.concatenate((np.asarray(cot_y, dtype), gd0, np.zeros_like(y)), axis=1)
    g = np.where(converged[:, None], g, 0).astype(dtype)
    lam, info, residual, iterations = batched_restarted_gmres(
        operator, g, tolerance=cfg.gmres_tolerance, absolute_tolerance=cfg.gmres_atol,
        restart=cfg.gmres_restart, max_iterations=cfg.gmres_max_iterations)
    valid = (converged & np.all(np.isfinite(lam), axis=1) & np.isfinite(residual)
             & ((info == 0) | (residual <= dtype.type(cfg.adjoint_tolerance))))
    lv = np.where(valid[:, None], lam, 0)
    pb = pullback(lin, lv[:, :n], lv[:, n:n + m], lv[:, n + m:])

    def clean(a):
        return np.nan_to_num(a, nan=0.0, posinf=0.0, neginf=0.0)

    return AdjointResult(clean(pb.g_values), clean(pb.g_rhs), clean(pb.g_target),
                         clean(pb.g_lower), clean(pb.g_upper), valid, info, residual, lam,
                         tau, sigma, None if pb.g_q is None else clean(pb.g_q), iterations)
