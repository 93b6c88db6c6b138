"""GPU parity with diagonal preconditioning (non-accelerated CP with per-row sigma
and per-variable tau; reference src/purin/solvers/chambolle_pock/kernels.py:76-88,
209-210, and the adjoint's steps in bounds.py:83-86).

The oracle's ``diagonal_step_sizes`` is pinned by the reference's metric bound
``||sqrt(S) K sqrt(T)||_2 <= safety`` (tests/test_oracle_cp.py); these tests hold
the HIP path to it at the fp64 / fp32 bars.
"""

import numpy as np
import pytest

from oracle import cp as ocp
from oracle import projection as op
from purin_amd import workloads
from tests._gpu import canonical_from_workload, plan_for, rel_err, require_gpu, to_np

pytestmark = pytest.mark.gpu

TOL = {np.float64: 1e-10, np.float32: 1e-4}


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("early_stop", [False, True])
def test_diagonal_solve_matches_oracle(dtype, early_stop):
    require_gpu()
    B = 50
    w = workloads.small_random(13, n=48, me=8, mi=20, width=4, batch=B)
    canon = canonical_from_workload(w)
    rhs = np.tile(w.rhs, (B, 1)).astype(dtype)
    target = w.target.astype(dtype)
    cfg = op.Config(diagonal_preconditioning=True)
    pre = op.presolve(canon, rhs, cfg, dtype)
    ksup, kmask = pre.support[pre.rows], pre.mask[pre.rows]
    iters = 400
    tol = 1e-6 if dtype == np.float64 else 1e-4
    want = ocp.sparse_cp(np.ones_like(target), -target, pre.kept_values[0], pre.kept_rhs, ksup,
                         kmask, canon.me, pre.lower, pre.upper, accelerated=False,
                         max_iterations=iters, tolerance=tol, y0=target,
                         freeze_converged=True, check_stationarity=True, norm_bound=True,
                         diagonal_preconditioning=True, early_stop=early_stop)
    plan = plan_for(canon, dtype=dtype, diagonal_preconditioning=True)
    got = plan.solve(pre.kept_rhs, target, pre.lower, pre.upper, tolerance=tol,
                     max_iterations=iters, early_stop=early_stop, check_every=5)
    bar = TOL[dtype]
    assert rel_err(to_np(got.y), want.y) <= bar
    assert rel_err(to_np(got.dual), want.dual) <= bar
    np.testing.assert_array_equal(to_np(got.iterations), want.iterations)
    np.testing.assert_array_equal(to_np(got.converged), want.converged)
    # the preconditioned steps differ from the scalar ones: the iterates must too
    scalar = ocp.sparse_cp(np.ones_like(target), -target, pre.kept_values[0], pre.kept_rhs, ksup,
                           kmask, canon.me, pre.lower, pre.upper, accelerated=False,
                           max_iterations=iters, tolerance=tol, y0=target,
                           freeze_converged=True, check_stationarity=True, norm_bound=True,
                           early_stop=early_stop)
    assert rel_err(scalar.y, want.y) > 1e-6
    y = to_np(got.y)
    lo, hi = np.broadcast_to(pre.lower, y.shape), np.broadcast_to(pre.upper, y.shape)
    np.testing.assert_array_equal(y == lo, want.y == lo)
    np.testing.assert_array_equal(y == hi, want.y == hi)
    np.testing.assert_array_equal(to_np(got.dual)[:, canon.me:] > 0, want.dual[:, canon.me:] > 0)


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_diagonal_project_matches_oracle(dtype):
    """Full projection (presolve, CP, dual recovery, statuses) at a fixed iteration count."""
    require_gpu()
    B = 33
    w = workloads.config1(batch=B)
    canon = canonical_from_workload(w)
    rhs = np.tile(w.rhs, (B, 1)).astype(dtype)
    target = w.target.astype(dtype)
    cfg = op.Config(diagonal_preconditioning=True, max_iterations=700, early_stop=False)
    want = op.solve(canon, target, rhs, cfg, dtype=dtype)
    plan = plan_for(canon, dtype=dtype, diagonal_preconditioning=True)
    got = plan.project(target, rhs, max_iterations=700, early_stop=False)
    bar = TOL[dtype]
    assert rel_err(to_np(got.y), want.y) <= bar
    np.testing.assert_array_equal(to_np(got.status), want.status)
    mult = to_np(got.multipliers)
    want_mult = np.concatenate([want.multipliers_eq, want.multipliers_ineq], axis=1)
    assert rel_err(mult, want_mult) <= TOL[dtype]


def test_diagonal_vjp_matches_oracle_at_the_same_state():
    """The adjoint linearises the preconditioned cp_step (per-row sigma, per-variable
    tau) at the GPU's converged state; converged GMRES at 1e-14."""
    from oracle import adjoint as oadj

    require_gpu()
    B = 40
    dtype = np.float64
    w = workloads.small_random(22, n=24, me=4, mi=8, width=3, batch=B)
    canon = canonical_from_workload(w)
    rhs = np.tile(w.rhs, (B, 1))
    target = w.target
    cot = np.random.default_rng(3).normal(size=(B, canon.n))
    cfg = op.Config(max_iterations=20000, tolerance=1e-9, diagonal_preconditioning=True,
                    gmres_tolerance=1e-14, gmres_max_iterations=300)
    pre = op.presolve(canon, rhs, cfg, dtype)
    plan = plan_for(canon, dtype=dtype, diagonal_preconditioning=True)
    o, saved = plan.solve(pre.kept_rhs, target, pre.lower, pre.upper, tol=pre.tolerance,
                          feasible=pre.feasible, max_iterations=cfg.max_iterations,
                          tolerance=cfg.tolerance, early_stop=True, save=True)
    conv = to_np(o.converged)
    assert conv.sum() >= B // 2
    ksup, kmask = pre.support[pre.rows], pre.mask[pre.rows]
    want = oadj.adjoint(pre.kept_values[0], ksup, kmask, canon.me, to_np(o.y), to_np(o.dual),
                        conv, target, pre.kept_rhs, pre.lower, pre.upper, cot, cfg)
    adj = plan.adjoint(saved, target, pre.kept_rhs, cot, bounds_grad=True, rhs_rows=plan.m,
                       tolerance=cfg.gmres_tolerance, max_iterations=cfg.gmres_max_iterations)
    np.testing.assert_array_equal(to_np(adj.valid), want.valid)
    np.testing.assert_array_equal(to_np(adj.info), want.info)
    assert rel_err(to_np(adj.g_target), want.g_target) <= 1e-10
    assert rel_err(to_np(adj.g_rhs), want.g_rhs) <= 1e-10
    assert rel_err(to_np(adj.g_lower), want.g_lower) <= 1e-10
    assert rel_err(to_np(adj.g_upper), want.g_upper) <= 1e-10


def test_diagonal_vjp_known_answer():
    """u + v == b, u >= 0 (reference tests/test_regression_chambolle_pock.py:26-56) with
    diagonal preconditioning: the same projection and Jacobian."""
    torch = require_gpu()
    from purin_amd.plan import Plan

    tiny = Plan(2, 1, 1, np.array([0, 2, 3]), np.array([0, 1, 0]), np.array([1.0, 1.0, -1.0]),
                dtype=torch.float64, diagonal_preconditioning=True, device="cuda")
    t_hat = np.array([[2.0, 0.0], [-2.0, 0.0]])
    t_rhs = np.array([[1.0, 0.0], [1.0, 0.0]])
    fwd = tiny.project(t_hat, t_rhs, save=True)
    np.testing.assert_allclose(to_np(fwd.y), [[1.5, -0.5], [0.0, 1.0]], atol=1e-8)
    jac = np.zeros((2, 2, 2))
    for k in range(2):
        cot = np.zeros((2, 2))
        cot[:, k] = 1.0
        jac[:, k, :] = to_np(tiny.adjoint(fwd.saved, None, None, cot).g_target)
    np.testing.assert_allclose(jac, [[[0.5, -0.5], [-0.5, 0.5]], [[0.0, 0.0], [0.0, 0.0]]],
                               atol=1e-8)
