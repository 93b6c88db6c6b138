"""Known-answer pins for the projection oracle (oracle/projection.py).

Each case restates an expected value from the reference's own tests (cited per
test); the reference itself cannot run here (JAX is absent).
"""

import numpy as np
import pytest

from oracle import projection as op
from oracle import qp as bf
from oracle.projection import Canonical, Config
from tests import _cases


def jacobian_target(canon, target, rhs, cfg, dtype=np.float64):
    """Rows of dy/dyhat and dy/drhs for every sample, one cotangent per output."""
    B, n = target.shape
    jt = np.zeros((B, n, n))
    jr = np.zeros((B, n, rhs.shape[1]))
    for k in range(n):
        cot = np.zeros((B, n))
        cot[:, k] = 1.0
        _, gt, gr, _ = op.vjp(canon, target, rhs, cfg, cot, dtype=dtype)
        jt[:, k, :] = gt
        jr[:, k, :] = gr
    return jt, jr


@pytest.mark.parametrize("accelerated", [False, True])
def test_affine_projection_and_gradients(accelerated):
    """Reference tests/test_regression_chambolle_pock.py:25-56."""
    canon = _cases.sum_equals_b_u_nonneg()
    cfg = Config(accelerated=accelerated)
    target = np.array([[2.0, 0.0], [-2.0, 0.0]])
    rhs = np.array([[1.0, 0.0], [1.0, 0.0]])
    out = op.solve(canon, target, rhs, cfg)
    np.testing.assert_allclose(out.y, [[1.5, -0.5], [0.0, 1.0]], atol=1e-8)
    assert np.all(out.status == op.CONVERGED)
    assert np.max(out.residual_inf_norm) <= cfg.tolerance
    jt, jr = jacobian_target(canon, target, rhs, cfg)
    np.testing.assert_allclose(jt[0], [[0.5, -0.5], [-0.5, 0.5]], atol=1e-8)
    np.testing.assert_allclose(jt[1], 0, atol=1e-8)
    np.testing.assert_allclose(jr[0][:, 0], [0.5, 0.5], atol=1e-8)
    np.testing.assert_allclose(jr[1][:, 0], [0.0, 1.0], atol=1e-8)
    eps = 1e-4
    fd = (op.solve(canon, target, rhs + [[eps, 0]], cfg).y
          - op.solve(canon, target, rhs - [[eps, 0]], cfg).y) / (2 * eps)
    np.testing.assert_allclose(fd, [[0.5, 0.5], [0.0, 1.0]], atol=1e-5)


def test_iteration_limit_and_nonfinite_diagnostics():
    """Reference tests/test_regression_chambolle_pock.py:68-85."""
    canon = _cases.sum_equals_b_u_nonneg()
    cfg = Config(max_iterations=1)
    target = np.array([[-2.0, 0.0]])
    rhs = np.array([[1.0, 0.0]])
    out = op.solve(canon, target, rhs, cfg)
    assert out.status[0] == op.MAX_ITERATIONS
    assert not out.gradient_eligible[0]
    _, gt, _, _ = op.vjp(canon, target, rhs, cfg, np.ones((1, 2)))
    np.testing.assert_allclose(gt, 0)
    out = op.solve(canon, np.array([[np.nan, 0.0]]), rhs, cfg)
    assert out.status[0] == op.NONFINITE


def test_no_constraints_is_identity_with_unit_gradient():
    """Reference tests/test_regression_chambolle_pock.py:88-95."""
    canon = Canonical(n=2, me=0, rows=[], coef=[])
    x = np.array([[0.2, 0.7]])
    rhs = np.zeros((1, 0))
    out = op.solve(canon, x, rhs, Config())
    np.testing.assert_allclose(out.y, x, atol=1e-12)
    _, gt, _, _ = op.vjp(canon, x, rhs, Config(), np.ones((1, 2)))
    np.testing.assert_allclose(gt, 1, atol=1e-9)


def test_inequality_only_with_warm_start():
    """Reference tests/test_regression_chambolle_pock.py:98-113."""
    canon = _cases.canonical_from_dense(np.zeros((0, 2)), [[-1.0, 0.0], [0.0, 1.0]], 2)
    out = op.solve(canon, np.array([[-2.0, 3.0]]), np.array([[0.0, 1.0]]), Config(),
                   multipliers_ineq=np.array([[0.2, 0.3]]))
    np.testing.assert_allclose(out.y, [[0.0, 1.0]], atol=1e-8)
    assert out.gradient_eligible[0]


def test_infeasible_problem_never_claims_convergence():
    """Reference tests/test_regression_chambolle_pock.py:140-153."""
    canon = _cases.canonical_from_dense(np.zeros((0, 1)), [[1.0], [-1.0]], 1)
    out = op.solve(canon, np.zeros((1, 1)), np.array([[0.0, -1.0]]), Config(max_iterations=100))
    assert out.status[0] == op.MAX_ITERATIONS
    assert not out.gradient_eligible[0]


def test_scaled_constraints_report_original_units():
    """Reference tests/test_regression_chambolle_pock.py:156-164."""
    canon = _cases.canonical_from_dense([[1000.0, 1000.0]], [[-1.0, 0.0]], 2)
    out = op.solve(canon, np.array([[2.0, 0.0]]), np.array([[1000.0, 0.0]]), Config())
    assert out.gradient_eligible[0]
    assert abs(np.sum(out.y) * 1000 - 1000) <= Config().tolerance


def test_tied_scaled_bounds_restore_duals_and_slacks():
    """Reference tests/test_regression_cp_bound_presolve.py:13-27."""
    canon, rhs = _cases.tied_scaled_bounds()
    out = op.solve(canon, np.array([[-3.0, 4.0]]), rhs[None], Config())
    np.testing.assert_allclose(out.y, [[0.0, 1.0]], atol=1e-10)
    np.testing.assert_allclose(out.multipliers_ineq, [[1.5, 0.75, 0.0, 3.0]], atol=1e-9)
    np.testing.assert_allclose(out.slacks, [[0.0, 0.0, 2.0, 0.0]], atol=1e-10)
    assert out.status[0] == op.CONVERGED
    assert len(op.presolve(canon, rhs[None], Config(), np.float64).rows) == 0
    _, gt, _, _ = op.vjp(canon, np.array([[-3.0, 4.0]]), rhs[None], Config(), np.ones((1, 2)))
    np.testing.assert_allclose(gt, 0.0, atol=1e-9)


@pytest.mark.parametrize("a,b,x,expected,eligible,g_b", [
    (2.0, 1.0, 3.0, 0.5, True, 0.5),
    (-2.0, 1.0, -3.0, -0.5, True, -0.5),
    (0.0, -1.0, 3.0, 3.0, False, 0.0),
    (0.0, 1.0, 3.0, 3.0, True, 0.0),
])
def test_parameter_dependent_bound_sign_and_zero(a, b, x, expected, eligible, g_b):
    """Reference tests/test_regression_cp_bound_presolve.py:30-53 (``a u <= b``).

    The derivative w.r.t. ``b`` is checked; the one w.r.t. ``a`` needs
    per-sample coefficients, which the shared-matrix path does not take.
    """
    canon = Canonical(n=1, me=0, rows=[[0]], coef=[[a]])
    out = op.solve(canon, np.array([[x]]), np.array([[b]]), Config())
    np.testing.assert_allclose(out.y, [[expected]], atol=1e-10)
    assert bool(out.gradient_eligible[0]) == eligible
    _, gt, gr, _ = op.vjp(canon, np.array([[x]]), np.array([[b]]), Config(), np.ones((1, 1)))
    np.testing.assert_allclose(gr, [[g_b]], atol=1e-8)
    if not eligible:
        np.testing.assert_allclose(gt, 0.0)


@pytest.mark.parametrize("seed", [12, 42])
def test_coupled_qp_matches_exact_projection_and_finite_difference(seed):
    """Reference tests/test_regression_cp_bound_presolve.py:56-109 (OSQP -> brute force)."""
    rng = np.random.default_rng(seed)
    canon, rhs = _cases.coupled_qp()
    x = rng.normal(size=(1, 3))
    out = op.solve(canon, x, rhs[None], Config())
    K = canon.dense()
    y_ref, lam_eq, lam_in = bf.project_bruteforce(x[0], K[:1], rhs[:1], K[1:], rhs[1:])
    np.testing.assert_allclose(out.y[0], y_ref, atol=2e-8)
    np.testing.assert_allclose(
        (out.y[0] - x[0]) + K.T @ np.r_[out.multipliers_eq[0], out.multipliers_ineq[0]],
        0.0, atol=1e-9)
    assert out.gradient_eligible[0]
    g = rng.normal(size=(1, 3))
    _, gt, _, _ = op.vjp(canon, x, rhs[None], Config(), g)
    for i in range(3):
        d = np.zeros_like(x)
        d[0, i] = 1e-4
        fd = np.sum((op.solve(canon, x + d, rhs[None], Config()).y
                     - op.solve(canon, x - d, rhs[None], Config()).y) * g) / 2e-4
        np.testing.assert_allclose(gt[0, i], fd, atol=2e-5)


def test_affine_projection_value_and_jacobian():
    """Reference tests/test_projections.py:65-75 and .github/scripts/numerical_regression.py:70-82."""
    canon = _cases.sum_equals_b()
    cfg = Config(tolerance=1e-9, max_iterations=3000)
    for dtype, atol in ((np.float64, 2e-6), (np.float32, 5e-5)):
        target = np.array([[0.8, 0.7]], dtype)
        rhs = np.ones((1, 1), dtype)
        out = op.solve(canon, target, rhs, cfg, dtype=dtype)
        assert out.y.dtype == dtype
        np.testing.assert_allclose(out.y, [[0.55, 0.45]], atol=atol)
    jt, _ = jacobian_target(canon, np.array([[0.8, 0.7]]), np.ones((1, 1)), cfg)
    np.testing.assert_allclose(jt[0], [[0.5, -0.5], [-0.5, 0.5]], atol=2e-5)


@pytest.mark.parametrize("accelerated", [False, True])
def test_projection_with_active_inequality(accelerated):
    """Reference tests/test_projections.py:78-97."""
    canon = _cases.sum_equals_b(inequalities=True)
    cfg = Config(accelerated=accelerated, tolerance=1e-9, max_iterations=3000)
    out = op.solve(canon, np.array([[2.0, -1.0]]), np.array([[1.0, 0.0, 0.0]]), cfg)
    np.testing.assert_allclose(out.y, [[1.0, 0.0]], atol=2e-6)


def weighted_solve(canon, diagonal, target, rhs, cfg):
    """Diagonal-metric change of variables; reference src/purin/solvers/metric.py:15-182."""
    diagonal = np.asarray(diagonal, np.float64)
    inverse = 1 / np.sqrt(diagonal)
    scaled = Canonical(canon.n, canon.me, canon.rows,
                       [[v * inverse[j] for j, v in zip(r, c)] for r, c in zip(canon.rows, canon.coef)])
    factor = max(1.0, float(np.sqrt(np.max(diagonal))))
    base = Config(**{**cfg.__dict__, "tolerance": cfg.tolerance / factor})
    root = np.sqrt(diagonal)
    out = op.solve(scaled, target * root, rhs, base)
    return out._replace(y=out.y / root, residual_inf_norm=out.residual_inf_norm * factor), scaled, base


def test_weighted_projection_value_and_jacobian():
    """Reference tests/test_projections.py:121-124 and tests/test_training_metric_contracts.py:63-83."""
    canon = _cases.sum_equals_b()
    out, scaled, base = weighted_solve(canon, [1.0, 4.0], np.array([[2.0, 0.0]]), np.ones((1, 1)),
                                       Config())
    np.testing.assert_allclose(out.y, [[1.2, -0.2]], atol=2e-6)
    root = np.sqrt([1.0, 4.0])
    jt, _ = jacobian_target(scaled, np.array([[2.0, 0.0]]) * root, np.ones((1, 1)), base)
    jac = jt[0] / root[:, None] * root[None, :]
    np.testing.assert_allclose(jac, [[0.2, -0.8], [-0.2, 0.8]], atol=2e-5)


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_random_projection_kkt_and_closed_form_jacobian(seed):
    """Converged outputs satisfy KKT and the gradients equal the closed-form active-set derivative."""
    canon, rhs, rng = _cases.random_canonical(seed, n=4, me=1, mi=2, width=3, bound=1.0)
    B = 3
    target = rng.normal(0, 1.5, (B, 4))
    rhs_b = np.tile(rhs, (B, 1))
    cfg = Config(tolerance=1e-11, max_iterations=200000)
    out = op.solve(canon, target, rhs_b, cfg)
    assert np.all(out.status == op.CONVERGED)
    K = canon.dense()
    me = canon.me
    jt, jr = jacobian_target(canon, target, rhs_b, cfg)
    for b in range(B):
        y, le, li = bf.project_bruteforce(target[b], K[:me], rhs[:me], K[me:], rhs[me:])
        np.testing.assert_allclose(out.y[b], y, atol=1e-9)
        assert bf.kkt_violation(out.y[b], target[b], out.multipliers_eq[b],
                                out.multipliers_ineq[b], K[:me], rhs[:me], K[me:], rhs[me:]) < 1e-8
        if np.any((li > 0) & (li < 1e-6)):
            continue  # near-degenerate: derivative not unique
        dyy, dyb, dyh = bf.active_set_jacobians(y, K[:me], K[me:], rhs[me:], li)
        np.testing.assert_allclose(jt[b], dyy, atol=1e-7)
        np.testing.assert_allclose(jr[b][:, :me], dyb, atol=1e-7)
        np.testing.assert_allclose(jr[b][:, me:], dyh, atol=1e-7)
