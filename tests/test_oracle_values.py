"""Pins for the oracle's per-sample coefficients (oracle/projection.py
``presolve``/``solve``/``vjp`` with ``values``).

The reference's parameter-dependent coefficient tests give known answers
(tests/test_regression_chambolle_pock.py:116-137,
tests/test_regression_cp_bound_presolve.py:30-53,
tests/test_regression_cp_diagonal_steps.py:83-112); central finite differences
of the exact projection (``oracle/qp.py``, active-set enumeration) pin the
coefficient gradient, including the row-scaling and bound-threshold chain.
"""

import numpy as np
import pytest

from oracle import projection as op
from oracle import qp as bf
from oracle.projection import Canonical, Config
from tests import _cases


def _affine_a(a):
    """``a u + v == 1``: one equality row with per-sample coefficients [a, 1]."""
    canon = Canonical(n=2, me=1, rows=[[0, 1]], coef=[[1.0, 1.0]])
    a = np.atleast_1d(np.asarray(a, np.float64))
    values = np.stack([np.stack([a, np.ones_like(a)], axis=1)], axis=1)  # (B, 1, 2)
    return canon, values


def _affine_expected(a, x):
    f = (a * x[0] + x[1] - 1) / (a * a + 1)
    y = x - np.array([a, 1.0]) * f
    fp = (x[0] * (a * a + 1) - (a * x[0] + x[1] - 1) * 2 * a) / (a * a + 1) ** 2
    dy_da = -np.array([f + a * fp, fp])
    return y, dy_da


def _jac_values(canon, target, rhs, cfg, values):
    """Per sample: d y / d values for every output (B, n, M, w)."""
    B, n = target.shape
    out = np.zeros((B, n) + values.shape[1:])
    for k in range(n):
        cot = np.zeros((B, n))
        cot[:, k] = 1.0
        res, _, _, _, gv = op.vjp(canon, target, rhs, cfg, cot, values=values, return_values=True)
        out[:, k] = gv
    return res, out


@pytest.mark.parametrize("accelerated,diagonal", [(False, False), (True, False), (False, True)])
def test_parameter_dependent_coefficient_known_answer(accelerated, diagonal):
    """Reference tests/test_regression_chambolle_pock.py:116-137 and
    tests/test_regression_cp_diagonal_steps.py:83-112: ``a u + v == 1``, a = 2."""
    x = np.array([0.2, 0.3])
    canon, values = _affine_a([2.0])
    cfg = Config(accelerated=accelerated, diagonal_preconditioning=diagonal)
    res, jac = _jac_values(canon, x[None], np.array([[1.0]]), cfg, values)
    y, dy_da = _affine_expected(2.0, x)
    np.testing.assert_allclose(res.y[0], y, atol=1e-8)
    np.testing.assert_allclose(jac[0, :, 0, 0], dy_da, atol=2e-7)


def test_parameter_dependent_bound_sign_zero_and_derivative():
    """Reference tests/test_regression_cp_bound_presolve.py:30-53: ``a u <= b``."""
    canon = Canonical(n=1, me=0, rows=[[0]], coef=[[1.0]])
    cfg = Config()

    def run(x, a, b):
        vals = np.array([[[a]]])
        return op.vjp(canon, np.array([[x]]), np.array([[b]]), cfg, np.ones((1, 1)),
                      values=vals, return_values=True)

    res, gt, gr, _, gv = run(3.0, 2.0, 1.0)
    np.testing.assert_allclose(res.y, [[0.5]], atol=1e-10)
    np.testing.assert_allclose([gv[0, 0, 0], gr[0, 0]], [-0.25, 0.5], atol=1e-8)
    res, *_ = run(-3.0, -2.0, 1.0)
    np.testing.assert_allclose(res.y, [[-0.5]], atol=1e-10)
    res, gt, gr, _, gv = run(3.0, 0.0, -1.0)  # 0 * u <= -1: infeasible
    assert not res.gradient_eligible[0]
    np.testing.assert_allclose(gt, 0.0)
    np.testing.assert_allclose(gv, 0.0)
    res, *_ = run(3.0, 0.0, 1.0)  # 0 * u <= 1: no bound
    np.testing.assert_allclose(res.y, [[3.0]])


def _random_case(seed, B=3):
    """n = 4: one equality, two coupled inequalities and a singleton bound row,
    per-sample coefficients, at a nondegenerate exact solution."""
    rng = np.random.default_rng(seed)
    rows = [[0, 1, 2, 3], [0, 2], [1, 3], [2]]
    canon = Canonical(n=4, me=1, rows=rows, coef=[[1.0] * len(r) for r in rows])
    w = max(len(r) for r in rows)
    values = np.zeros((B, 4, w))
    for i, r in enumerate(rows):
        values[:, i, : len(r)] = rng.uniform(0.5, 2.0, (B, len(r))) * rng.choice([-1, 1], (B, len(r)))
    values[:, 3, 0] = rng.uniform(0.5, 2.0, B)  # bound row c u_2 <= h with c > 0
    target = rng.normal(size=(B, 4)) * 2
    rhs = rng.uniform(-0.5, 0.5, (B, 4))
    rhs[:, 1:] = np.abs(rhs[:, 1:]) * 0.2
    return canon, values, target, rhs


def _dense(canon, vals):
    A = np.zeros((len(canon.rows), canon.n))
    for i, r in enumerate(canon.rows):
        A[i, r] = vals[i, : len(r)]
    return A


def _exact(canon, vals, yhat, rhs):
    A = _dense(canon, vals)
    y, _, lam = bf.project_bruteforce(yhat, A[: canon.me], rhs[: canon.me], A[canon.me:],
                                      rhs[canon.me:])
    return y, lam, A


@pytest.mark.parametrize("seed", [3, 11])
@pytest.mark.parametrize("row_scaling", [True, False])
def test_coefficient_gradient_matches_exact_projection_differences(seed, row_scaling):
    """g_values (CP fixed point + GMRES adjoint + presolve chain) against central
    differences of the exact projection in every coefficient."""
    canon, values, target, rhs = _random_case(seed)
    B = target.shape[0]
    cfg = Config(tolerance=1e-12, max_iterations=200000, row_scaling=row_scaling,
                 gmres_tolerance=1e-13, gmres_max_iterations=200)
    cot = np.random.default_rng(seed + 1).normal(size=target.shape)
    res, _, g_rhs, _, gv = op.vjp(canon, target, rhs, cfg, cot, values=values,
                                  return_values=True)
    assert np.all(res.status == op.CONVERGED)
    h = 1e-6
    for b in range(B):
        y, lam, A = _exact(canon, values[b], target[b], rhs[b])
        np.testing.assert_allclose(res.y[b], y, atol=1e-9)
        # nondegenerate: active rows have clearly positive multipliers
        slack = rhs[b, canon.me:] - A[canon.me:] @ y
        assert np.all((lam > 1e-4) | (slack > 1e-4))
        for i, r in enumerate(canon.rows):
            for s in range(len(r)):
                vp = values[b].copy()
                vm = values[b].copy()
                vp[i, s] += h
                vm[i, s] -= h
                fd = (_exact(canon, vp, target[b], rhs[b])[0]
                      - _exact(canon, vm, target[b], rhs[b])[0]) / (2 * h)
                np.testing.assert_allclose(gv[b, i, s], cot[b] @ fd, atol=2e-6,
                                           err_msg=f"sample {b} row {i} slot {s}")
        for i in range(len(canon.rows)):
            rp = rhs[b].copy()
            rm = rhs[b].copy()
            rp[i] += h
            rm[i] -= h
            fd = (_exact(canon, values[b], target[b], rp)[0]
                  - _exact(canon, values[b], target[b], rm)[0]) / (2 * h)
            np.testing.assert_allclose(g_rhs[b, i], cot[b] @ fd, atol=2e-6)


def test_shared_values_reduce_to_the_shared_path():
    """Per-sample values equal to the shared coefficients give the shared result."""
    canon, rhs = _cases.coupled_qp()
    _, _, shared = canon.ell(np.float64)
    target = np.array([[0.9, 0.6, 0.8], [2.0, -1.0, 0.1]])
    rhs_b = np.tile(rhs, (2, 1))
    cfg = Config(max_iterations=400, early_stop=False)
    a = op.solve(canon, target, rhs_b, cfg)
    b = op.solve(canon, target, rhs_b, cfg, values=np.broadcast_to(shared, (2,) + shared.shape))
    np.testing.assert_allclose(b.y, a.y, rtol=0, atol=1e-13)
    np.testing.assert_array_equal(b.status, a.status)


@pytest.mark.parametrize("row_scaling", [True, False])
def test_row_scaling_pullback_matches_finite_differences(row_scaling):
    """The presolve chain alone: the gradient of
    ``<G, s(K) K> + <g, s(K) r>`` w.r.t. ``K`` and ``r`` by central differences.
    (At an exact projection the ``s^3`` term vanishes, because the projection is
    invariant to scaling a row and its rhs together; this pins it directly.)"""
    rng = np.random.default_rng(5)
    B, m, w = 2, 3, 4
    mask = np.array([[1, 1, 1, 0], [1, 1, 0, 0], [1, 1, 1, 1]], bool)
    K = np.where(mask, rng.normal(size=(B, m, w)), 0)
    r = rng.normal(size=(B, m))
    G = np.where(mask, rng.normal(size=(B, m, w)), 0)
    g = rng.normal(size=(B, m))

    def f(K, r):
        norms = np.sqrt(np.sum(K ** 2, axis=2))
        s = 1 / norms if row_scaling else np.ones_like(norms)
        return np.sum(G * K * s[:, :, None]) + np.sum(g * r * s)

    gK, gr = op.row_scaling_pullback(K, mask, r, G, g, row_scaling)
    h = 1e-6
    for idx in zip(*np.nonzero(np.broadcast_to(mask, K.shape))):
        Kp, Km = K.copy(), K.copy()
        Kp[idx] += h
        Km[idx] -= h
        np.testing.assert_allclose(gK[idx], (f(Kp, r) - f(Km, r)) / (2 * h), atol=1e-8)
    for idx in np.ndindex(r.shape):
        rp, rm = r.copy(), r.copy()
        rp[idx] += h
        rm[idx] -= h
        np.testing.assert_allclose(gr[idx], (f(K, rp) - f(K, rm)) / (2 * h), atol=1e-8)
