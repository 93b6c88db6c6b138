"""Pins for the adjoint restatement (oracle/adjoint.py)."""

import numpy as np
import pytest

from oracle import adjoint as adj
from oracle import cp
from tests import _cases


def _random_state(seed, n=6, m=5, me=2, B=3, diagonal=False):
    """A random CP state; ``diagonal`` gives per-variable tau and per-row sigma
    (diagonal preconditioning, kernels.py:76-88)."""
    rng = np.random.default_rng(seed)
    K = rng.normal(size=(m, n)) * (rng.uniform(size=(m, n)) < 0.6)
    support, mask = cp.layout([tuple(np.flatnonzero(r)) for r in K], n)
    values = cp.ell_values(K, support, mask)
    y = rng.uniform(-1.5, 1.5, (B, n))
    dual = rng.normal(size=(B, m))
    target = rng.normal(size=(B, n))
    rhs = rng.normal(size=(B, m))
    lower, upper = -np.ones((B, n)), np.ones((B, n))
    tau, sigma = np.full(B, 0.3), np.full(B, 0.4)
    if diagonal:
        tau, sigma = rng.uniform(0.1, 0.5, (B, n)), rng.uniform(0.1, 0.5, (B, m))
    return values, support, mask, me, y, dual, target, rhs, lower, upper, tau, sigma, rng


def _step(values, support, mask, me, z, target, rhs, lower, upper, tau, sigma, n, m):
    mv, tmv = cp.operators(values, support, mask, n)
    y, d, yb = z[:, :n], z[:, n:n + m], z[:, n + m:]
    out = cp.cp_step((y, d, yb), np.ones_like(target), -target, rhs, lower, upper, mv, tmv, me,
                     tau, sigma, np.ones(y.shape[0]))
    return np.concatenate(out, axis=1)


@pytest.mark.parametrize("diagonal", [False, True])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_pullback_matches_finite_differences(seed, diagonal):
    """The mask-form VJP equals the transpose of the finite-difference Jacobian of cp_step."""
    values, support, mask, me, y, dual, target, rhs, lower, upper, tau, sigma, rng = _random_state(
        seed, diagonal=diagonal)
    B, n = y.shape
    m = dual.shape[1]
    lin = adj.linearize(values, support, mask, me, y, dual, target, rhs, lower, upper, tau, sigma)
    z0 = np.concatenate((y, dual, y), axis=1)
    W = z0.shape[1]
    cot = rng.normal(size=(B, W))
    pb = adj.pullback(lin, cot[:, :n], cot[:, n:n + m], cot[:, n + m:])
    eps = 1e-6
    f = lambda z: _step(values, support, mask, me, z, target, rhs, lower, upper, tau, sigma, n, m)
    # state directions (the linearisation point has ybar = y, so perturb all three blocks)
    for k in range(W):
        dz = np.zeros_like(z0)
        dz[:, k] = eps
        jcol = (f(z0 + dz) - f(z0 - dz)) / (2 * eps)
        expect = np.sum(jcol * cot, axis=1)
        got = np.concatenate((pb.gy, pb.gd, pb.gbar), axis=1)[:, k]
        np.testing.assert_allclose(got, expect, atol=1e-7)
    # rhs, target, bound directions
    for name, arr, grad in (("rhs", rhs, pb.g_rhs), ("target", target, pb.g_target),
                            ("lower", lower, pb.g_lower), ("upper", upper, pb.g_upper)):
        for k in range(arr.shape[1]):
            d = np.zeros_like(arr)
            d[:, k] = eps
            args = dict(rhs=rhs, target=target, lower=lower, upper=upper)
            args[name] = arr + d
            fp = _step(values, support, mask, me, z0, args["target"], args["rhs"], args["lower"],
                       args["upper"], tau, sigma, n, m)
            args[name] = arr - d
            fm = _step(values, support, mask, me, z0, args["target"], args["rhs"], args["lower"],
                       args["upper"], tau, sigma, n, m)
            np.testing.assert_allclose(grad[:, k], np.sum((fp - fm) / (2 * eps) * cot, axis=1),
                                       atol=1e-7, err_msg=name)


@pytest.mark.parametrize("diagonal", [False, True])
def test_pullback_coefficient_gradient_matches_finite_differences(diagonal):
    values, support, mask, me, y, dual, target, rhs, lower, upper, tau, sigma, rng = _random_state(
        5, diagonal=diagonal)
    B, n = y.shape
    m = dual.shape[1]
    lin = adj.linearize(values, support, mask, me, y, dual, target, rhs, lower, upper, tau, sigma)
    z0 = np.concatenate((y, dual, y), axis=1)
    cot = rng.normal(size=z0.shape)
    pb = adj.pullback(lin, cot[:, :n], cot[:, n:n + m], cot[:, n + m:])
    eps = 1e-6
    for i in range(support.shape[0]):
        for s in range(support.shape[1]):
            if not mask[i, s]:
                continue
            vp = np.broadcast_to(values, (B,) + values.shape).copy()
            vm = vp.copy()
            vp[:, i, s] += eps
            vm[:, i, s] -= eps
            fp = _step(vp, support, mask, me, z0, target, rhs, lower, upper, tau, sigma, n, m)
            fm = _step(vm, support, mask, me, z0, target, rhs, lower, upper, tau, sigma, n, m)
            np.testing.assert_allclose(pb.g_values[:, i, s],
                                       np.sum((fp - fm) / (2 * eps) * cot, axis=1), atol=1e-7)


@pytest.mark.parametrize("restart,max_it", [(30, 100), (3, 60), (40, 40)])
def test_gmres_matches_dense_solve(restart, max_it):
    rng = np.random.default_rng(3)
    B, W = 4, 12
    mats = np.eye(W)[None] * 2 + 0.3 * rng.normal(size=(B, W, W))
    rhs = rng.normal(size=(B, W))
    x, info, res, _ = adj.batched_restarted_gmres(
        lambda v: np.einsum("bij,bj->bi", mats, v), rhs, tolerance=1e-12,
        absolute_tolerance=0.0, restart=restart, max_iterations=max_it)
    exact = np.linalg.solve(mats, rhs[:, :, None])[:, :, 0]
    assert np.all(info == 0)
    np.testing.assert_allclose(x, exact, atol=1e-10)
    assert np.all(res <= 1e-12 * np.abs(rhs).max(axis=1))


def test_gmres_reports_nonconvergence_and_zero_rhs():
    rng = np.random.default_rng(4)
    B, W = 2, 20
    mats = np.eye(W)[None] + 0.9 * rng.normal(size=(B, W, W))
    rhs = rng.normal(size=(B, W))
    rhs[1] = 0.0
    x, info, res, _ = adj.batched_restarted_gmres(
        lambda v: np.einsum("bij,bj->bi", mats, v), rhs, tolerance=1e-14,
        absolute_tolerance=0.0, restart=2, max_iterations=4)
    assert info[0] == 1 and res[0] > 0
    assert info[1] == 0 and np.all(x[1] == 0)


def test_adjoint_independent_of_step_sizes():
    """Fixed-point invariance: the converged gradient does not depend on tau/sigma."""
    from oracle import projection as op

    canon, rhs = _cases.coupled_qp()
    x = np.array([[0.9, -0.2, 0.8]])
    cfg = op.Config(tolerance=1e-11, max_iterations=100000)
    res, out, pre = op.solve(canon, x, rhs[None], cfg, return_internal=True)
    ksup, kmask = pre.support[pre.rows], pre.mask[pre.rows]
    g = np.array([[0.3, -1.0, 0.5]])
    grads = []
    m = len(pre.rows)
    diag = (np.array([[0.1, 0.3, 0.2]]), np.linspace(0.15, 0.45, m)[None])  # per-variable / row
    for steps in (None, (np.array([0.05]), np.array([0.2])), (np.array([0.4]), np.array([0.5])),
                  diag):
        a = adj.adjoint(pre.kept_values, ksup, kmask, canon.me, out.y, out.dual, out.converged,
                        x, pre.kept_rhs, pre.lower, pre.upper, g, cfg, steps=steps)
        assert a.valid[0]
        grads.append(a.g_target)
    np.testing.assert_allclose(grads[1], grads[0], atol=1e-8)
    np.testing.assert_allclose(grads[2], grads[0], atol=1e-8)
    np.testing.assert_allclose(grads[3], grads[0], atol=1e-8)
