"""Pins for the dense-adapter oracle (oracle/dense.py).

The reference's known answers (tests/test_dense_cp.py:20-73), a dense
nonsymmetric system for the BiCGSTAB restatement, and exact QP solutions
(``oracle/qp.py`` after ``z = sqrt(q) y``) with their central differences for
the implicit gradient.
"""

import numpy as np
import pytest

from oracle import dense as od
from oracle import qp as bf

Q = np.array([[2.0, 4.0]])
C_LIN = np.array([[-2.0, -4.0]])
A = np.ones((1, 1, 2))
B = np.ones((1, 1))
G = np.array([[[-1.0, 0.0]]])
D = np.zeros((1, 1))
LO = np.zeros((1, 2))
HI = np.ones((1, 2)) * 2


@pytest.mark.parametrize("accelerated", [False, True])
@pytest.mark.parametrize("equilibrate", [False, True])
def test_dense_cp_matches_analytic_equality_qp(accelerated, equilibrate):
    """Reference tests/test_dense_cp.py:20-49 (values, warm start, dy/dc)."""
    kw = dict(accelerated=accelerated, equilibrate=equilibrate, tolerance=1e-13,
              max_iterations=20000)
    y, lam, mu, it, out = od.solve_dense(Q, C_LIN, A, B, G, D, LO, HI, **kw)
    np.testing.assert_allclose(y, [[1 / 3, 2 / 3]], atol=1e-6)
    warm = od.solve_dense(Q, C_LIN, A, B, G, D, LO, HI, y0=y, lambda0=lam, mu0=mu, **kw)
    np.testing.assert_allclose(warm[0], y, atol=1e-6)
    if equilibrate:
        return  # the derivative through the equilibration is the front end's (autograd)
    values = np.concatenate((A, G), axis=1)
    rhs = np.concatenate((B, D), axis=1)
    jac = np.zeros((2, 2))
    for k in range(2):
        cot = np.zeros((1, 2))
        cot[0, k] = 1.0
        g_c, *_ = od.implicit_vjp(Q, C_LIN, values, rhs, LO, HI, 1, out.y, out.dual, cot,
                                  np.zeros((1, 2)))
        jac[k] = g_c[0]
    expected = -np.diag([0.5, 0.25]) + np.outer([0.5, 0.25], [0.5, 0.25]) / 0.75
    np.testing.assert_allclose(jac, expected, atol=1e-6)


def test_dense_empty_constraints():
    """Reference tests/test_dense_cp.py:52-73."""
    y, *_ = od.solve_dense(np.ones((1, 2)), np.array([[-1.0, -2.0]]), np.zeros((1, 0, 2)),
                           np.zeros((1, 0)), np.zeros((1, 0, 2)), np.zeros((1, 0)),
                           np.zeros((1, 2)), np.ones((1, 2)) * 3, equilibrate=True,
                           tolerance=1e-14)
    np.testing.assert_allclose(y, [[1.0, 2.0]], atol=1e-6)


def test_bicgstab_solves_a_nonsymmetric_system():
    rng = np.random.default_rng(0)
    M = np.eye(12) * 3 + rng.normal(size=(12, 12)) * 0.3
    b = rng.normal(size=12)
    x, k = od.bicgstab(lambda v: M @ v, b, tol=1e-13, maxiter=200)
    np.testing.assert_allclose(M @ x, b, atol=1e-11)
    assert 0 < k < 200
    x0, k0 = od.bicgstab(lambda v: M @ v, np.zeros(12), tol=1e-6, maxiter=50)
    assert k0 == 0 and not np.any(x0)


def _exact(q, c, A_, b, G_, d, lo, hi):
    s = np.sqrt(q)
    n = q.size
    fin_hi, fin_lo = np.isfinite(hi), np.isfinite(lo)
    Gz = np.vstack((G_ / s, np.eye(n)[fin_hi], -np.eye(n)[fin_lo]))
    h = np.concatenate((d, (hi * s)[fin_hi], (-lo * s)[fin_lo]))
    z, _, lam = bf.project_bruteforce(-c / s, A_ / s, b, Gz, h)
    return z / s, lam, h - Gz @ z


def test_implicit_gradient_matches_exact_differences():
    """The frozen-prox fixed-point VJP (BiCGSTAB at 1e-13) against central
    differences of the exact QP in c, the matrix entries, the rhs and the bounds."""
    rng = np.random.default_rng(11)
    n, me, mi = 3, 1, 2
    q = rng.uniform(0.5, 2.5, (1, n))
    c = rng.normal(size=(1, n))
    A_ = rng.normal(size=(1, me, n))
    G_ = rng.normal(size=(1, mi, n))
    x0 = rng.uniform(-0.3, 0.3, (1, n))
    b = np.einsum("bmn,bn->bm", A_, x0)
    d = np.einsum("bmn,bn->bm", G_, x0) + np.array([[0.05, 0.6]])
    lo, hi = np.full((1, n), -0.7), np.full((1, n), 0.7)
    y, lam, mu, it, out = od.solve_dense(q, c, A_, b, G_, d, lo, hi, tolerance=1e-12,
                                         max_iterations=400000)
    ye, lame, slack = _exact(q[0], c[0], A_[0], b[0], G_[0], d[0], lo[0], hi[0])
    np.testing.assert_allclose(y[0], ye, atol=1e-9)
    assert np.all((lame > 1e-4) | (slack > 1e-4)), "degenerate case"
    cot = rng.normal(size=(1, n))
    values = np.concatenate((A_, G_), axis=1)
    rhs = np.concatenate((b, d), axis=1)
    g_c, g_v, g_r, g_lo, g_hi, k = od.implicit_vjp(q, c, values, rhs, lo, hi, me, out.y,
                                                   out.dual, cot, np.zeros((1, me + mi)),
                                                   tolerance=1e-13, adjoint_iterations=500)
    assert k > 0
    h = 1e-6

    def f(**kw):
        args = dict(q=q[0], c=c[0], A_=A_[0], b=b[0], G_=G_[0], d=d[0], lo=lo[0], hi=hi[0])
        args.update(kw)
        return cot[0] @ _exact(**args)[0]

    def diff(name, arr, idx):
        up, dn = arr.copy(), arr.copy()
        up[idx] += h
        dn[idx] -= h
        return (f(**{name: up}) - f(**{name: dn})) / (2 * h)

    for j in range(n):
        np.testing.assert_allclose(g_c[0, j], diff("c", c[0], j), atol=2e-6)
        np.testing.assert_allclose(g_lo[0, j], diff("lo", lo[0], j), atol=2e-6)
        np.testing.assert_allclose(g_hi[0, j], diff("hi", hi[0], j), atol=2e-6)
    for i in range(me):
        np.testing.assert_allclose(g_r[0, i], diff("b", b[0], i), atol=2e-6)
        for j in range(n):
            np.testing.assert_allclose(g_v[0, i, j], diff("A_", A_[0], (i, j)), atol=2e-6)
    for i in range(mi):
        np.testing.assert_allclose(g_r[0, me + i], diff("d", d[0], i), atol=2e-6)
        for j in range(n):
            np.testing.assert_allclose(g_v[0, me + i, j], diff("G_", G_[0], (i, j)), atol=2e-6)
