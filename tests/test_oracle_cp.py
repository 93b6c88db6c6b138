"""Pins for the CP kernel restatement (oracle/cp.py) independent of its own formulas."""

import numpy as np
import pytest

from oracle import cp
from oracle import qp as bf
from tests import _cases


@pytest.mark.parametrize("rows", [((0, 1), (1, 2)), ((0,), (0, 1, 2), (2,)), ()])
def test_layout_products_match_dense(rows):
    """Reference tests/test_sparse_layouts.py:15-51: ELL products equal a dense einsum."""
    support, mask = cp.layout(rows, 3)
    values = (np.arange(2 * support.size, dtype=np.float64).reshape((2,) + support.shape) + 1) * mask
    vector = np.arange(2 * len(rows), dtype=np.float64).reshape((2, len(rows))) + 1
    dense = np.zeros((2, len(rows), 3))
    for r, idx in enumerate(rows):
        for s, c in enumerate(idx):
            dense[:, r, c] = values[:, r, s]
    np.testing.assert_allclose(cp.tmatvec(values, support, mask, vector, 3),
                               np.einsum("bmn,bm->bn", dense, vector))
    x = np.arange(6, dtype=np.float64).reshape(2, 3)
    np.testing.assert_allclose(cp.matvec(values, support, mask, x),
                               np.einsum("bmn,bn->bm", dense, x))


def test_proximal_closed_form_and_cache():
    """Reference tests/test_regression_cp_proximal_coefficients.py:11-53."""
    rng = np.random.default_rng(42)
    q = rng.uniform(0.1, 5.0, (3, 7))
    c = rng.normal(size=(3, 7))
    tau = np.array([0.1, 0.4, 0.7])
    y = rng.normal(size=(3, 7))
    a, d, offset = cp.proximal_coefficients(q, c, tau)
    np.testing.assert_allclose(a * y - d * (2 * y) + offset,
                               (y - tau[:, None] * (2 * y + c)) / (1 + tau[:, None] * q),
                               atol=1e-14)
    q = np.array([[0.0, 0.3, 2.0]])
    c = np.array([[1.0, -1.0, 0.5]])
    y = np.array([[0.3, 0.2, -0.1]])
    dual = np.array([[0.2, 0.3, 0.4]])
    tau, sigma, theta = np.array([0.3]), np.array([0.2]), np.ones(1)
    args = ((y, dual, y), q, c, np.zeros_like(y), np.full_like(y, -2.0), np.full_like(y, 2.0),
            lambda x: x, lambda x: x, 1, tau, sigma, theta)
    uncached = cp.cp_step(*args)
    cached = cp.cp_step(*args, proximal=cp.proximal_coefficients(q, c, tau))
    for u, v in zip(cached, uncached):
        np.testing.assert_array_equal(u, v)


def test_diagonal_steps_metric_bound():
    """Reference tests/test_regression_cp_diagonal_steps.py:13-26."""
    matrix = np.array([[100.0, 0.0, 0.2, 0.0], [0.0, 0.01, 0.0, 0.0], [0.0, 0.0, 0.0, 0.0]])
    support, mask = cp.layout([tuple(np.flatnonzero(r)) for r in matrix], 4)
    values = cp.ell_values(matrix, support, mask)
    tau, sigma = cp.diagonal_step_sizes(np.ones((2, 4)), values, support, mask, 0.95)
    assert np.all(np.isfinite(tau)) and np.all(tau > 0)
    assert np.all(np.isfinite(sigma)) and np.all(sigma > 0)
    for t, s in zip(tau, sigma):
        assert np.linalg.norm(np.sqrt(s)[:, None] * matrix * np.sqrt(t)[None, :], 2) <= 0.95 + 1e-14


def test_norm_bound_closed_form_and_power_iteration():
    rng = np.random.default_rng(7)
    K = rng.normal(size=(5, 9)) * (rng.uniform(size=(5, 9)) < 0.4)
    support, mask = cp.layout([tuple(np.flatnonzero(r)) for r in K], 9)
    values = cp.ell_values(K, support, mask)
    expected = np.sqrt(np.abs(K).sum(1).max() * np.abs(K).sum(0).max())
    np.testing.assert_allclose(cp.norm_bound(values, support, mask, 2, 9, np.float64), expected,
                               rtol=1e-15)
    mv, tmv = cp.operators(values, support, mask, 9)
    est = cp.norm_estimate(mv, tmv, 2, 9, np.float64, iterations=200)
    two = np.linalg.norm(K, 2)
    assert np.all(est <= two * (1 + 1e-12) + 1e-12)
    np.testing.assert_allclose(est, two, rtol=1e-6)
    # 20 iterations (the default) gives a lower estimate within a few percent here
    est20 = cp.norm_estimate(mv, tmv, 1, 9, np.float64)
    assert 0.9 * two <= est20[0] <= two * (1 + 1e-12)


def test_start_vector_is_deterministic_and_spread():
    v = cp.start_vector(1000, 42, np.float64)
    np.testing.assert_array_equal(v, cp.start_vector(1000, 42, np.float64))
    assert -1 <= v.min() < -0.9 and 0.9 < v.max() < 1
    assert abs(v.mean()) < 0.1
    assert not np.array_equal(v, cp.start_vector(1000, 43, np.float64))


@pytest.mark.parametrize("accelerated", [False, True])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_sparse_cp_converges_to_bruteforce_projection(accelerated, seed):
    """A converged CP solve equals the exact projection (replaces the reference's OSQP check).

    The accelerated variant's stationarity decays like 1/k (tau_k -> 0), so it
    is checked at a looser tolerance.
    """
    rng = np.random.default_rng(100 + seed)
    n, me, mi = 5, 1, 3
    K = rng.normal(size=(me + mi, n)) * (rng.uniform(size=(me + mi, n)) < 0.7)
    K[:, 0] += 0.5
    x0 = rng.uniform(-0.3, 0.3, n)
    rhs = K @ x0
    rhs[me:] += rng.uniform(0.1, 0.5, mi)
    support, mask = cp.layout([tuple(np.flatnonzero(r)) for r in K], n)
    values = cp.ell_values(K, support, mask)
    batch = 4
    yhat = rng.normal(0, 1.5, (batch, n))
    lower, upper = -np.ones((batch, n)), np.ones((batch, n))
    out = cp.sparse_cp(np.ones_like(yhat), -yhat, values, np.tile(rhs, (batch, 1)), support,
                       mask, me, lower, upper, accelerated=accelerated, max_iterations=100000,
                       tolerance=1e-8 if accelerated else 1e-11, y0=yhat, freeze_converged=True,
                       check_stationarity=True, norm_bound=True)
    assert accelerated or np.all(out.converged)
    A_in = np.vstack((K[me:], np.eye(n), -np.eye(n)))
    h = np.concatenate((rhs[me:], np.ones(n), np.ones(n)))
    for b in range(batch):
        y_ref, lam_eq, lam_in = bf.project_bruteforce(yhat[b], K[:me], rhs[:me], A_in, h)
        np.testing.assert_allclose(out.y[b], y_ref, atol=1e-6 if accelerated else 1e-9)


def test_fixed_iteration_mode_runs_every_iteration():
    canon = _cases.sum_equals_b()
    support, mask, values = canon.ell(np.float64)
    yhat = np.array([[0.8, 0.7], [2.0, 0.0]])
    out = cp.sparse_cp(np.ones_like(yhat), -yhat, values, np.ones((2, 1)), support, mask, 1,
                       -np.inf * np.ones_like(yhat), np.inf * np.ones_like(yhat),
                       max_iterations=37, tolerance=1e-3, y0=yhat, freeze_converged=True,
                       check_stationarity=True, norm_bound=True, early_stop=False)
    np.testing.assert_array_equal(out.iterations, [37, 37])
    early = cp.sparse_cp(np.ones_like(yhat), -yhat, values, np.ones((2, 1)), support, mask, 1,
                         -np.inf * np.ones_like(yhat), np.inf * np.ones_like(yhat),
                         max_iterations=37, tolerance=1e-3, y0=yhat, freeze_converged=True,
                         check_stationarity=True, norm_bound=True)
    assert np.all(early.iterations < 37)


def _schedule_violations(sched, tau0, sigma0, gamma):
    """Which relations fixed by the accelerated update (kernels.py:279-283:
    nu = 1/sqrt(1 + gamma tau), tau <- nu tau, sigma <- sigma/nu, theta <- nu)
    a schedule ``(tau_k, sigma_k, theta_k)`` breaks."""
    tau, sigma, theta = (np.asarray(c, np.float64) for c in np.asarray(sched).T)
    k = np.arange(len(tau), dtype=np.float64)
    bad = []
    if not (tau[0] == tau0 and sigma[0] == sigma0 and theta[0] == 1.0):
        bad.append("start")
    # the step product tau sigma is invariant (sigma is divided by what tau is multiplied by)
    if not np.allclose(tau * sigma, tau0 * sigma0, rtol=1e-12, atol=0):
        bad.append("tau*sigma")
    # theta_{k+1} is the factor that took tau_k to tau_{k+1}
    if not np.allclose(theta[1:], tau[1:] / tau[:-1], rtol=1e-14, atol=0):
        bad.append("theta")
    # squaring nu: 1/tau_{k+1}^2 = 1/tau_k^2 + gamma/tau_k
    if not np.allclose(1 / tau[1:] ** 2 - 1 / tau[:-1] ** 2, gamma / tau[:-1], rtol=1e-9, atol=0):
        bad.append("recursion")
    # hence 1/tau_k grows like gamma k / 2: gamma tau_k k -> 2
    if not abs(gamma * tau[-1] * k[-1] - 2.0) < 1e-2:
        bad.append("asymptote")
    return bad


@pytest.mark.parametrize("gamma", [1.0, 0.25, 3.0])
def test_accelerated_schedule_invariants(gamma):
    """Pins ``accelerated_schedule`` by what the recurrence fixes, not by restating
    it: the invariant step product, theta as the step ratio, the squared
    recursion and the 2/(gamma k) decay (20000 steps)."""
    tau0, sigma0 = 0.3, 0.2
    sched = cp.accelerated_schedule(tau0, sigma0, 20000, np.float64, gamma=gamma)
    assert _schedule_violations(sched, tau0, sigma0, gamma) == []
    s32 = cp.accelerated_schedule(tau0, sigma0, 5, np.float32, gamma=gamma)
    assert s32.dtype == np.float32


def test_schedule_invariants_reject_planted_mistakes():
    """Each plausible slip in the update fails at least one relation: sigma
    multiplied instead of divided, a doubled gamma, theta the inverse factor."""
    tau0, sigma0, gamma = 0.3, 0.2, 1.0

    def planted(kind, iters=20000):
        out = np.empty((iters, 3))
        tau, sigma, theta = tau0, sigma0, 1.0
        for k in range(iters):
            out[k] = (tau, sigma, theta)
            nu = 1 / np.sqrt(1 + (2 * gamma if kind == "2gamma" else gamma) * tau)
            tau = nu * tau
            sigma = sigma * nu if kind == "sigma" else sigma / nu
            theta = 1 / nu if kind == "theta" else nu
        return out

    assert _schedule_violations(planted("none"), tau0, sigma0, gamma) == []
    assert "tau*sigma" in _schedule_violations(planted("sigma"), tau0, sigma0, gamma)
    assert {"recursion", "asymptote"} <= set(_schedule_violations(planted("2gamma"), tau0,
                                                                  sigma0, gamma))
    assert "theta" in _schedule_violations(planted("theta"), tau0, sigma0, gamma)


def test_sparse_cp_takes_the_schedule_steps(monkeypatch):
    """The accelerated loop of ``sparse_cp`` updates its steps through
    ``accelerated_update`` once per iteration, so it walks exactly the
    ``accelerated_schedule`` pinned above."""
    canon = _cases.sum_equals_b()
    support, mask, values = canon.ell(np.float64)
    yhat = np.array([[0.8, 0.7], [2.0, 0.0]])
    q = np.ones_like(yhat)
    inf = np.inf * np.ones_like(yhat)
    seen = []
    real = cp.accelerated_update

    def spy(tau, sigma, gamma):
        seen.append((np.array(tau, copy=True), np.array(sigma, copy=True), np.array(gamma)))
        return real(tau, sigma, gamma)

    monkeypatch.setattr(cp, "accelerated_update", spy)
    cp.sparse_cp(q, -yhat, values, np.ones((2, 1)), support, mask, 1, -inf, inf,
                 accelerated=True, max_iterations=7, y0=yhat, freeze_converged=True,
                 check_stationarity=True, norm_bound=True, early_stop=False)
    monkeypatch.setattr(cp, "accelerated_update", real)
    assert len(seen) == 7
    tau0, sigma0 = seen[0][0][0], seen[0][1][0]
    sched = cp.accelerated_schedule(tau0, sigma0, 7, np.float64)
    for k, (tau, sigma, gamma) in enumerate(seen):
        np.testing.assert_array_equal(gamma, [1.0, 1.0])  # gamma = min q
        np.testing.assert_array_equal(tau, [sched[k, 0]] * 2)
        np.testing.assert_array_equal(sigma, [sched[k, 1]] * 2)
