"""NumPy restatement of PURIN's dense CP adapter and its implicit layer.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows ``src/purin/solvers/chambolle_pock/dense.py:26-105`` (``solve_dense``:
the shared CP iteration with dense operators, ``factored_proximal=True``, no
freezing, no stationarity test, power-iteration steps), the equilibration of
``src/purin/linalg/equilibration.py:21-57`` (Ruiz) as used by
``dense_layer.py:13-134``, and the implicit backward of
``dense_implicit.py:63-238`` with ``src/purin/autodiff/fixed_point.py:8-40``:
BiCGSTAB on ``(I - J_z^T) v = cot`` over the whole flattened batch (tolerance
1e-6, ``adjoint_iters`` iterations), the step sizes and the prox inverse
frozen, so there is no derivative through ``q``.

The BiCGSTAB is JAX's ``jax.scipy.sparse.linalg.bicgstab`` (jax 0.6.2, the
version PURIN's CI pins; not vendored in the reference): preconditioned
BiCGSTAB (van der Vorst 1992) with ``rho = alpha = omega = 1``,
``rhat = p = q = r0 = b`` initially, the early exit when ``|s|^2 < atol2``,
breakdown codes when ``rho``, ``alpha`` or ``omega`` vanish, and
``atol2 = max(tol^2 |b|^2, atol^2)``; restated here from that published
algorithm.

Pinned by: the reference's known answers (tests/test_dense_cp.py:20-73:
``[1/3, 2/3]``, ``dy/dc``, the empty-constraint case) and exact QP solutions
with their central differences (tests/test_oracle_dense.py).
"""

from __future__ import annotations

import numpy as np

from oracle import adjoint as _adj
from oracle import cp as _cp


def dense_layout(n, me, mi):
    """Every row on all n columns: the ELL support of a dense matrix."""
    rows = [list(range(n))] * (me + mi)
    return _cp.layout(rows, n)


def ruiz_equilibrate(q, c, A, b, C, d, lower, upper, iterations=4, eps=1e-6):
    """equilibration.py:21-57: alternate column and row scaling by 1/sqrt(max|.|)."""
    dtype = q.dtype
    columns = np.ones_like(q)
    eqs, iqs = np.ones_like(b), np.ones_like(d)
    epsilon = dtype.type(eps)
    one = dtype.type(1)
    for _ in range(iterations):
        colA = np.max(np.abs(A), axis=1) if A.shape[1] else np.zeros_like(q)
        colC = np.max(np.abs(C), axis=1) if C.shape[1] else np.zeros_like(q)
        metric = np.maximum(np.maximum(colA, colC), np.abs(q))
        update = one / np.sqrt(np.maximum(metric, epsilon))
        A, C = A * update[:, None, :], C * update[:, None, :]
        q, c = q * (update ** 2), c * update
        lower, upper, columns = lower / update, upper / update, columns * update
        if A.shape[1]:
            update = one / np.sqrt(np.maximum(np.max(np.abs(A), axis=2), epsilon))
            A, b, eqs = A * update[:, :, None], b * update, eqs * update
        if C.shape[1]:
            update = one / np.sqrt(np.maximum(np.max(np.abs(C), axis=2), epsilon))
            C, d, iqs = C * update[:, :, None], d * update, iqs * update
    return q, c, A, b, C, d, lower, upper, columns, eqs, iqs


def solve_dense(q, c, A, b, C, d, lower, upper, *, accelerated=False, safety=0.95,
                norm_iterations=20, norm_seed=42, max_iterations=5000, tolerance=1e-9,
                y0=None, lambda0=None, mu0=None, equilibrate=False,
                equilibration_iterations=10, trace=None):
    """dense_layer.py:76-134 with dense.py:26-105.  Returns (y, lambda, mu, iterations)."""
    q = np.asarray(q)
    dtype = q.dtype
    c, A, b, C, d = (np.asarray(x, dtype) for x in (c, A, b, C, d))
    batch, n = q.shape
    A = np.broadcast_to(A, (batch,) + A.shape[-2:]) if A.ndim == 2 else A
    C = np.broadcast_to(C, (batch,) + C.shape[-2:]) if C.ndim == 2 else C
    me, mi = A.shape[1], C.shape[1]
    b, d = np.broadcast_to(b, (batch, me)), np.broadcast_to(d, (batch, mi))
    lower = np.broadcast_to(np.asarray(lower, dtype), (batch, n))
    upper = np.broadcast_to(np.asarray(upper, dtype), (batch, n))
    y0 = np.zeros((batch, n), dtype) if y0 is None else np.asarray(y0, dtype)
    lam0 = np.zeros((batch, me), dtype) if lambda0 is None else np.asarray(lambda0, dtype)
    mu0 = np.zeros((batch, mi), dtype) if mu0 is None else np.asarray(mu0, dtype)
    columns, eqs, iqs = np.ones_like(q), np.ones_like(b), np.ones_like(d)
    if equilibrate:
        q, c, A, b, C, d, lower, upper, columns, eqs, iqs = ruiz_equilibrate(
            q, c, A, b, C, d, lower, upper, iterations=equilibration_iterations)
        y0 = y0 / columns
        lam0 = lam0 / np.where(eqs == 0.0, 1.0, eqs)
        mu0 = mu0 / np.where(iqs == 0.0, 1.0, iqs)
    support, mask = dense_layout(n, me, mi)
    values = np.concatenate((A, C), axis=1)
    out = _cp.sparse_cp(q, c, values, np.concatenate((b, d), axis=1), support, mask, me, lower,
                        upper, accelerated=accelerated, safety=safety,
                        max_iterations=max_iterations, tolerance=tolerance,
                        norm_iterations=norm_iterations, norm_seed=norm_seed, y0=y0,
                        dual0=np.concatenate((lam0, mu0), axis=1), freeze_converged=False,
                        check_stationarity=False, norm_bound=False, factored_proximal=True,
                        trace=trace)
    return (columns * out.y, eqs * out.dual[:, :me], iqs * out.dual[:, me:], out.iterations,
            out)


def bicgstab(matvec, b, *, tol, atol=0.0, maxiter):
    """BiCGSTAB of jax.scipy.sparse.linalg (jax 0.6.2) on one flattened vector.

    Returns ``(x, k)`` with ``k`` the iterations run, or the breakdown code
    (-10: rho = 0, -11: omega or alpha = 0).
    """
    dtype = b.dtype
    bs = np.dot(b, b)
    atol2 = max(dtype.type(tol) ** 2 * bs, dtype.type(atol) ** 2)
    x = np.zeros_like(b)
    r = b - matvec(x)
    rhat, p, q = r.copy(), r.copy(), r.copy()
    rho = alpha = omega = dtype.type(1)
    k = 0
    while np.dot(r, r) > atol2 and k < maxiter and k >= 0:
        rho_ = np.dot(rhat, r)
        beta = rho_ / rho * alpha / omega
        p = r + beta * (p - omega * q)
        q = matvec(p)
        alpha_ = rho_ / np.dot(rhat, q)
        s = r - alpha_ * q
        exit_early = np.dot(s, s) < atol2
        t = matvec(s)
        omega_ = np.dot(t, s) / np.dot(t, t)
        if exit_early:
            x = x + alpha_ * p
            r = s
        else:
            x = x + (alpha_ * p + omega_ * s)
            r = s - omega_ * t
        k = -11 if (omega_ == 0 or alpha_ == 0) else k + 1
        k = -10 if rho_ == 0 else k
        rho, alpha, omega = rho_, alpha_, omega_
    return x, k


def dense_steps(q, values, support, mask, *, safety, norm_iterations, norm_seed):
    """dense_implicit.py:85-104: power-iteration L, tau = s/(max q + L), sigma = s/L."""
    dtype = q.dtype
    batch, n = q.shape
    mv, tmv = _cp.operators(values, support, mask, n)
    L = np.maximum(_cp.norm_estimate(mv, tmv, batch, n, dtype, norm_iterations, norm_seed),
                   dtype.type(1e-12))
    s = dtype.type(safety)
    return (s / (np.max(q, axis=1) + L)).astype(dtype), (s / L).astype(dtype)


def implicit_vjp(q, c, values, rhs, lower, upper, me, y, dual, cot_y, cot_dual, *, safety=0.95,
                 norm_iterations=20, norm_seed=42, tolerance=1e-6, adjoint_iterations=50):
    """The dense layer's backward on the (equilibrated) data it solved:
    ``fixed_point_pullback`` of the factored step at ``z = (y, dual, y)`` with
    frozen ``tau, sigma, theta = 1, inverse = 1/(1 + tau q)``.

    Returns ``(g_c, g_values, g_rhs, g_lower, g_upper, k)``; ``g_q`` is zero.
    """
    dtype = y.dtype
    batch, n = y.shape
    m = dual.shape[1]
    support, mask = dense_layout(n, me, m - me)
    tau, sigma = dense_steps(q, values, support, mask, safety=safety,
                             norm_iterations=norm_iterations, norm_seed=norm_seed)
    lin = _adj.linearize(values, support, mask, me, y, dual, None, rhs, lower, upper, tau, sigma,
                         q=q, c=c, factored_proximal=True)
    W = 2 * n + m

    def unflat(v):
        v = v.reshape(batch, W)
        return v[:, :n], v[:, n:n + m], v[:, n + m:]

    def matvec(v):
        gy, gd, gb = unflat(v)
        pb = _adj.pullback(lin, gy, gd, gb)
        return v - np.concatenate((pb.gy, pb.gd, pb.gbar), axis=1).ravel()

    # the reference flattens (y, equality, inequality, extrapolated) leaf by
    # leaf; the dot products are sums over the same entries in another order
    cot = np.concatenate((cot_y, cot_dual, np.zeros_like(y)), axis=1)
    sol, k = bicgstab(matvec, cot.ravel().astype(dtype), tol=tolerance, maxiter=adjoint_iterations)
    gy, gd, gb = unflat(sol)
    pb = _adj.pullback(lin, gy, gd, gb)
    return -pb.g_target, np.where(mask[None], pb.g_values, 0), pb.g_rhs, pb.g_lower, pb.g_upper, k
