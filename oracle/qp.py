"""Exact Euclidean projections onto small polyhedra, independent of CP.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

``project_bruteforce`` enumerates active sets of the inequality rows and
returns the unique KKT point of

    min 0.5 ||y - yhat||^2  s.t.  A_eq y = b,  A_in y <= h.

It replaces the reference's OSQP checks (reference
tests/test_regression_cp_bound_presolve.py:57-109,
tests/test_regression_cp_diagonal_steps.py:28-81), which cannot run here.

``active_set_jacobians`` is the closed-form derivative at a nondegenerate
solution: with ``Bm`` the equality rows plus the strictly active inequality
rows, ``dy/dyhat = I - Bm^T (Bm Bm^T)^+ Bm`` and
``dy/drhs_B = Bm^T (Bm Bm^T)^+`` (zero for inactive rows).

``kkt_violation`` measures stationarity, primal feasibility, dual sign and
complementarity, which characterise the projection uniquely.
"""

from __future__ import annotations

import itertools

import numpy as np


def _eq_projection(yhat, Bm, rb):
    """Project yhat onto {Bm y = rb}; returns y and multipliers (least-norm)."""
    if Bm.shape[0] == 0:
        return yhat.copy(), np.zeros(0)
    gram = Bm @ Bm.T
    lam = np.linalg.lstsq(gram, Bm @ yhat - rb, rcond=None)[0]
    return yhat - Bm.T @ lam, lam


def project_bruteforce(yhat, A_eq, b, A_in, h, tol=1e-11):
    """Exact projection by active-set enumeration (tiny problems only)."""
    yhat = np.asarray(yhat, np.float64)
    A_eq = np.asarray(A_eq, np.float64).reshape(-1, yhat.size)
    A_in = np.asarray(A_in, np.float64).reshape(-1, yhat.size)
    b = np.asarray(b, np.float64).reshape(-1)
    h = np.asarray(h, np.float64).reshape(-1)
    mi = A_in.shape[0]
    if mi > 16:
        raise ValueError("brute force is limited to 16 inequality rows")
    best = None
    for size in range(mi + 1):
        for active in itertools.combinations(range(mi), size):
            active = list(active)
            Bm = np.vstack((A_eq, A_in[active]))
            rb = np.concatenate((b, h[active]))
            y, lam = _eq_projection(yhat, Bm, rb)
            if Bm.shape[0] and np.max(np.abs(Bm @ y - rb)) > 1e-9:
                continue
            if mi and np.max(A_in @ y - h) > 1e-9:
                continue
            mu = lam[A_eq.shape[0]:]
            if mu.size and np.min(mu) < -tol:
                continue
            dist = np.sum((y - yhat) ** 2)
            if best is None or dist < best[0] - 1e-14:
                lam_eq = lam[: A_eq.shape[0]]
                lam_in = np.zeros(mi)
                lam_in[active] = mu
                best = (dist, y, lam_eq, lam_in)
    if best is None:
        raise ValueError("infeasible")
    return best[1], best[2], best[3]


def active_set_jacobians(y, A_eq, A_in, h, lam_in, tol=1e-9):
    """Closed-form ``dy/dyhat``, ``dy/db`` and ``dy/dh`` at a nondegenerate solution."""
    n = y.size
    A_eq = np.asarray(A_eq, np.float64).reshape(-1, n)
    A_in = np.asarray(A_in, np.float64).reshape(-1, n)
    active = [i for i in range(A_in.shape[0]) if lam_in[i] > tol]
    Bm = np.vstack((A_eq, A_in[active]))
    if Bm.shape[0]:
        pinv = np.linalg.pinv(Bm @ Bm.T)
        dy_dyhat = np.eye(n) - Bm.T @ pinv @ Bm
        dy_drb = Bm.T @ pinv
    else:
        dy_dyhat = np.eye(n)
        dy_drb = np.zeros((n, 0))
    dy_db = dy_drb[:, : A_eq.shape[0]]
    dy_dh = np.zeros((n, A_in.shape[0]))
    dy_dh[:, active] = dy_drb[:, A_eq.shape[0]:]
    return dy_dyhat, dy_db, dy_dh


def kkt_violation(y, yhat, lam_eq, lam_in, A_eq, b, A_in, h):
    """Max violation of the projection's KKT conditions."""
    n = y.size
    A_eq = np.asarray(A_eq, np.float64).reshape(-1, n)
    A_in = np.asarray(A_in, np.float64).reshape(-1, n)
    stat = y - yhat + A_eq.T @ lam_eq + A_in.T @ lam_in
    parts = [np.abs(stat).max(initial=0.0)]
    if A_eq.shape[0]:
        parts.append(np.abs(A_eq @ y - b).max())
    if A_in.shape[0]:
        r = A_in @ y - h
        parts.append(np.maximum(r, 0).max())
        parts.append(np.maximum(-lam_in, 0).max())
        parts.append(np.abs(lam_in * r).max())
    return max(parts)
