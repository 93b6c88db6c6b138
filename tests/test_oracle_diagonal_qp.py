"""Pins for the diagonal-QP oracle (oracle/diagonal_qp.py).

The reference's known answer (tests/test_diagonal_qp.py:13-48) and exact QP
solutions: with ``z = sqrt(q) y`` the QP ``min 0.5 y'Qy + c'y`` is the
projection of ``-c/sqrt(q)`` onto the scaled polyhedron, which
``oracle/qp.py`` solves by active-set enumeration; central differences of that
exact solution pin every gradient (q, c, values, rhs, lower, upper, and the
dual cotangent's path).
"""

import numpy as np
import pytest

from oracle import diagonal_qp as dq
from oracle import qp as bf
from oracle.cp import layout
from oracle.projection import CONVERGED, Config


@pytest.mark.parametrize("accelerated", [False, True])
@pytest.mark.parametrize("scaling", [False, True])
def test_diagonal_qp_value_and_coefficient_gradient(accelerated, scaling):
    """Reference tests/test_diagonal_qp.py:13-48."""
    rows, me, data = dq.dense_qp_data([[2.0, 4.0]], [[-2.0, -4.0]], np.ones((1, 2)), [1.0],
                                      np.empty((0, 2)), np.empty(0), -np.inf, np.inf)
    support, mask = layout(rows, 2)
    cfg = Config(accelerated=accelerated, row_scaling=scaling, tolerance=1e-9,
                 max_iterations=3000)
    res = dq.solve(support, mask, me, data, cfg)
    np.testing.assert_allclose(res.y, [[1 / 3, 2 / 3]], atol=1e-8)
    assert res.residual_inf_norm[0] < 1e-8
    expected = -np.diag([0.5, 0.25]) + np.outer([0.5, 0.25], [0.5, 0.25]) / 0.75
    jac = np.zeros((2, 2))
    for k in range(2):
        cot = np.zeros((1, 2))
        cot[0, k] = 1.0
        _, g, _ = dq.vjp(support, mask, me, data, cfg, cot)
        jac[k] = g.c[0]
    np.testing.assert_allclose(jac, expected, atol=1e-7)
    warm = dq.solve(support, mask, me, data, cfg, y0=res.y, dual0=res.multipliers_eq)
    np.testing.assert_allclose(warm.y, res.y, atol=1e-8)


def _exact(rows, me, n, q, c, vals, rhs, lo, hi):
    """Exact diagonal-QP solution and multipliers via z = sqrt(q) y."""
    A = np.zeros((len(rows), n))
    for i, r in enumerate(rows):
        A[i, r] = vals[i, : len(r)]
    s = np.sqrt(q)
    As = A / s[None, :]
    fin_hi, fin_lo = np.isfinite(hi), np.isfinite(lo)
    G = np.vstack((As[me:], np.eye(n)[fin_hi], -np.eye(n)[fin_lo]))
    h = np.concatenate((rhs[me:], (hi * s)[fin_hi], (-lo * s)[fin_lo]))
    z, _, lam = bf.project_bruteforce(-c / s, As[:me], rhs[:me], G, h)
    slack = h - G @ z
    return z / s, lam, slack


def _random_qp(seed, B=2):
    rng = np.random.default_rng(seed)
    n, me = 3, 1
    rows = [[0, 1, 2], [0, 1], [1, 2]]
    support, mask = layout(rows, n)
    values = np.where(mask[None], rng.uniform(0.5, 1.5, (B,) + mask.shape)
                      * rng.choice([-1, 1], (B,) + mask.shape), 0)
    q = rng.uniform(0.5, 3.0, (B, n))
    c = rng.normal(size=(B, n)) * 2
    x0 = rng.uniform(-0.3, 0.3, (B, n))
    rhs = np.einsum("bmw,bmw->bm", values, x0[:, support])
    rhs[:, me:] += rng.uniform(0.1, 0.5, (B, len(rows) - me))
    lower = np.tile([-0.6, -np.inf, -0.6], (B, 1))
    upper = np.tile([0.6, 0.6, np.inf], (B, 1))
    return rows, me, n, support, mask, dq.QPData(q, c, values, rhs, lower, upper)


def _multipliers(rows, me, n, q, c, vals, rhs, lo, hi):
    """Exact multipliers of the general rows in the reference's order: the
    inequality ones from the enumeration (z-space rows keep their multipliers),
    the equality ones from stationarity q y + c + K' lambda = 0 on the free
    variables."""
    y, lam, _ = _exact(rows, me, n, q, c, vals, rhs, lo, hi)
    m = len(rows)
    A = np.zeros((m, n))
    for i, r in enumerate(rows):
        A[i, r] = vals[i, : len(r)]
    lam_in = lam[: m - me]
    grad = q * y + c + A[me:].T @ lam_in
    free = (y > lo + 1e-9) & (y < hi - 1e-9)
    lam_eq = np.linalg.lstsq(A[:me].T[free], -grad[free], rcond=None)[0]
    return np.concatenate((lam_eq, lam_in))


def _check_against_differences(rows, me, n, data, b, g, f):
    """Every gradient of sample b against central differences of f(**inputs)."""
    h = 1e-6
    base = dict(q=data.q[b], c=data.c[b], vals=data.values[b], rhs=data.rhs[b],
                lo=data.lower[b], hi=data.upper[b])
    names = {"q": "q", "c": "c", "rhs": "rhs", "lower": "lo", "upper": "hi"}
    for name, key in names.items():
        arr = base[key]
        for j in range(arr.size):
            if not np.isfinite(arr[j]):
                continue
            up, dn = arr.copy(), arr.copy()
            up[j] += h
            dn[j] -= h
            want = (f(**{**base, key: up}) - f(**{**base, key: dn})) / (2 * h)
            np.testing.assert_allclose(getattr(g, name)[b, j], want, atol=3e-6,
                                       err_msg=f"{name}[{b},{j}]")
    for i, r in enumerate(rows):
        for s in range(len(r)):
            up, dn = base["vals"].copy(), base["vals"].copy()
            up[i, s] += h
            dn[i, s] -= h
            want = (f(**{**base, "vals": up}) - f(**{**base, "vals": dn})) / (2 * h)
            np.testing.assert_allclose(g.values[b, i, s], want, atol=3e-6,
                                       err_msg=f"values[{b},{i},{s}]")


@pytest.mark.parametrize("mode,seed", [("scalar", 1), ("scalar", 7), ("diagonal", 1),
                                       ("diagonal", 7), ("accelerated", 1), ("accelerated", 3)])
def test_qp_solution_and_gradients_match_exact_differences(seed, mode):
    """y against the exact QP; g_q, g_c, g_values, g_rhs, g_lower, g_upper against
    differences of cot . y (cot_dual = 0) and of cot_dual . multipliers (cot_y = 0)."""
    rows, me, n, support, mask, data = _random_qp(seed)
    B = data.q.shape[0]
    m = len(rows)
    cfg = Config(tolerance=1e-10, max_iterations=100000, gmres_tolerance=1e-13,
                 gmres_max_iterations=300, accelerated=mode == "accelerated",
                 diagonal_preconditioning=mode == "diagonal")
    rng = np.random.default_rng(seed + 100)
    cot = rng.normal(size=(B, n))
    cot_dual = rng.normal(size=(B, m))
    res, g, _ = dq.vjp(support, mask, me, data, cfg, cot)
    _, gd, _ = dq.vjp(support, mask, me, data, cfg, np.zeros((B, n)), cot_dual)
    assert np.all(res.status == CONVERGED)
    for b in range(B):
        y, lam, slack = _exact(rows, me, n, data.q[b], data.c[b], data.values[b], data.rhs[b],
                               data.lower[b], data.upper[b])
        np.testing.assert_allclose(res.y[b], y, atol=1e-9)
        assert np.all((lam > 1e-4) | (slack > 1e-4)), "degenerate case"
        mult = np.concatenate((res.multipliers_eq[b], res.multipliers_ineq[b]))
        np.testing.assert_allclose(mult, _multipliers(rows, me, n, data.q[b], data.c[b],
                                                      data.values[b], data.rhs[b],
                                                      data.lower[b], data.upper[b]), atol=1e-8)
        _check_against_differences(
            rows, me, n, data, b, g,
            lambda **kw: cot[b] @ _exact(rows, me, n, **kw)[0])
        _check_against_differences(
            rows, me, n, data, b, gd,
            lambda **kw: cot_dual[b] @ _multipliers(rows, me, n, **kw))
