"""Small canonical problems shared by the oracle and GPU tests.

Each case is written in PURIN's canonical sign convention (reference
src/purin/problems/expressions.py:298-309): ``a <= b`` becomes ``a - b <= 0``
and ``a >= b`` becomes ``b - a <= 0``; ``rhs = -g(theta, 0)``.
"""

from __future__ import annotations

import numpy as np

from oracle.projection import Canonical


def canonical_from_dense(A_eq, A_in, n):
    """Rows with ascending columns (reference problems/problem.py:358-364)."""
    rows, coef = [], []
    for mat in (A_eq, A_in):
        mat = np.asarray(mat, np.float64).reshape(-1, n)
        for r in mat:
            cols = np.flatnonzero(r)
            rows.append(cols.tolist())
            coef.append(r[cols].tolist())
    me = np.asarray(A_eq).reshape(-1, n).shape[0]
    return Canonical(n=n, me=me, rows=rows, coef=coef)


def sum_equals_b(inequalities=False):
    """``u + v == b`` (+ ``u >= 0``, ``v >= 0``); reference tests/test_projections.py:33-46."""
    A_eq = [[1.0, 1.0]]
    A_in = [[-1.0, 0.0], [0.0, -1.0]] if inequalities else np.zeros((0, 2))
    return canonical_from_dense(A_eq, A_in, 2)


def sum_equals_b_u_nonneg():
    """``u + v == b, u >= 0``; reference tests/test_regression_chambolle_pock.py:16-22."""
    return canonical_from_dense([[1.0, 1.0]], [[-1.0, 0.0]], 2)


def tied_scaled_bounds():
    """``u >= 0, 2u >= 0, u <= 2, v <= 1``; reference tests/test_regression_cp_bound_presolve.py:13-17."""
    A_in = [[-1.0, 0.0], [-2.0, 0.0], [1.0, 0.0], [0.0, 1.0]]
    rhs = np.array([0.0, 0.0, 2.0, 1.0])
    return canonical_from_dense(np.zeros((0, 2)), A_in, 2), rhs


def coupled_qp():
    """``u+v+w == 1, u >= 0, v >= -0.5, w <= 0.7, 2u - v <= 0.9``.

    Reference tests/test_regression_cp_bound_presolve.py:56-109.
    """
    A_eq = [[1.0, 1.0, 1.0]]
    A_in = [[-1.0, 0.0, 0.0], [0.0, -1.0, 0.0], [0.0, 0.0, 1.0], [2.0, -1.0, 0.0]]
    rhs = np.array([1.0, 0.0, 0.5, 0.7, 0.9])
    return canonical_from_dense(A_eq, A_in, 3), rhs


def random_canonical(seed, n, me, mi, width, bound):
    """Random sparse rows with box bounds as singleton rows and a feasible rhs."""
    rng = np.random.default_rng(seed)
    rows, coef = [], []
    for _ in range(me + mi):
        cols = np.sort(rng.choice(n, width, replace=False))
        rows.append(cols.tolist())
        coef.append(rng.normal(0.0, 1.0, width).tolist())
    x0 = rng.uniform(-0.5 * bound, 0.5 * bound, n)
    canon = Canonical(n=n, me=me, rows=rows, coef=coef)
    K = canon.dense()
    rhs = list(K[:me] @ x0) + list(K[me:] @ x0 + rng.uniform(0.0, 1.0, mi))
    for j in range(n):
        rows.append([j]); coef.append([1.0]); rhs.append(bound)
    for j in range(n):
        rows.append([j]); coef.append([-1.0]); rhs.append(bound)
    return canon, np.asarray(rhs), rng


def split_dense(canon):
    """Dense ``(A_eq, A_in)`` of a canonical problem."""
    K = canon.dense()
    return K[: canon.me], K[canon.me:]
