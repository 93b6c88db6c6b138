"""The reference's public-API CP tests, run through this build's front end on the GPU.

Each test restates a reference test (cited) with the reference's expected
values; gradients use torch autograd, whose backward is purin_cp_adjoint.
"""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as _torch

    if not _torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return _torch


def problem():
    from purin_amd import Projection

    p = Projection(method="chambolle-pock")
    t = p.add_parameter(["b"])
    y = p.add_variable(["u", "v"])
    p.objective = 0.0
    p.constraints.add(y.u + y.v == t.b, y.u >= 0)
    return p


def jac(torch, f, x):
    return torch.autograd.functional.jacobian(f, x).cpu().numpy()


@pytest.mark.parametrize("accelerated", [False, True])
def test_affine_projection_and_gradients(torch, accelerated):
    """Reference tests/test_regression_chambolle_pock.py:25-56."""
    from purin_amd import ChambollePockConfig, ImplicitGradientConfig, SolveStatus, prepare_projection

    cfg = ChambollePockConfig(
        accelerated=accelerated,
        implicit_gradient=ImplicitGradientConfig(differentiate_problem_parameters=True))
    layer = prepare_projection(problem(), method="chambolle-pock", config=cfg, batch_size=2)
    values = torch.tensor([[2.0, 0.0], [-2.0, 0.0]], dtype=torch.float64, device="cuda")
    theta = torch.ones((2, 1), dtype=torch.float64, device="cuda")
    out = layer.solve(values, theta)
    np.testing.assert_allclose(out.y.detach().cpu(), [[1.5, -0.5], [0.0, 1.0]], atol=1e-8)
    assert np.all(out.status.cpu().numpy() == int(SolveStatus.CONVERGED))
    assert float(out.residual_inf_norm.max()) <= cfg.tolerance
    j = jac(torch, lambda x: layer(x, theta), values)
    np.testing.assert_allclose(j[0, :, 0, :], [[0.5, -0.5], [-0.5, 0.5]], atol=1e-8)
    np.testing.assert_allclose(j[1, :, 1, :], 0, atol=1e-8)
    np.testing.assert_allclose(j[0, :, 1, :], 0, atol=1e-8)
    d = jac(torch, lambda t: layer(values, t), theta)
    np.testing.assert_allclose(d[0, :, 0, 0], [0.5, 0.5], atol=1e-8)
    np.testing.assert_allclose(d[1, :, 1, 0], [0.0, 1.0], atol=1e-8)
    eps = 1e-4
    fd = ((layer(values, theta + eps) - layer(values, theta - eps)) / (2 * eps)).detach().cpu()
    np.testing.assert_allclose(fd, [[0.5, 0.5], [0.0, 1.0]], atol=1e-5)


def test_rejects_nonlinear_constraints(torch):
    """Reference tests/test_regression_chambolle_pock.py:59-65."""
    from purin_amd import Projection, prepare_projection

    p = Projection()
    y = p.add_variable(["u"])
    p.objective = 0.0
    p.constraints.add(y.u ** 2 <= 1)
    with pytest.raises(ValueError, match="affine"):
        prepare_projection(p, method="chambolle-pock", batch_size=1)


def test_iteration_limit_and_nonfinite_diagnostics(torch):
    """Reference tests/test_regression_chambolle_pock.py:68-85."""
    from purin_amd import ChambollePockConfig, SolveStatus, prepare_projection

    layer = prepare_projection(problem(), method="chambolle-pock",
                               config=ChambollePockConfig(max_iterations=1), batch_size=1)
    one = torch.ones((1, 1), dtype=torch.float64)
    out = layer.solve(torch.tensor([[-2.0, 0.0]], dtype=torch.float64), one)
    assert int(out.status[0]) == int(SolveStatus.MAX_ITERATIONS)
    assert not bool(out.gradient_eligible[0])
    x = torch.tensor([[-2.0, 0.0]], dtype=torch.float64, device="cuda", requires_grad=True)
    layer(x, one).sum().backward()
    np.testing.assert_allclose(x.grad.cpu(), 0)
    out = layer.solve(torch.tensor([[float("nan"), 0.0]], dtype=torch.float64), one)
    assert int(out.status[0]) == int(SolveStatus.NONFINITE)


def test_no_constraints_and_unit_gradient(torch):
    """Reference tests/test_regression_chambolle_pock.py:88-95."""
    from purin_amd import Projection, prepare_projection

    p = Projection()
    p.add_variable(["u", "v"])
    p.objective = 0.0
    layer = prepare_projection(p, method="chambolle-pock", batch_size=1)
    x = torch.tensor([[0.2, 0.7]], dtype=torch.float64, device="cuda", requires_grad=True)
    np.testing.assert_allclose(layer(x).detach().cpu(), [[0.2, 0.7]], atol=1e-12)
    layer(x).sum().backward()
    np.testing.assert_allclose(x.grad.cpu(), 1, atol=1e-9)


def test_inequality_only_and_warm_start_gradients(torch):
    """Reference tests/test_regression_chambolle_pock.py:98-113."""
    from purin_amd import Projection, prepare_projection

    p = Projection()
    y = p.add_variable(["u", "v"])
    p.objective = 0.0
    p.constraints.add(y.u >= 0, y.v <= 1)
    layer = prepare_projection(p, method="chambolle-pock", batch_size=1)
    x = torch.tensor([[-2.0, 3.0]], dtype=torch.float64)
    out = layer.project_training(x, multipliers_ineq=torch.tensor([[0.2, 0.3]]))
    np.testing.assert_allclose(out.y_tilde.detach().cpu(), [[0.0, 1.0]], atol=1e-8)
    assert bool(out.forward_gradient_eligible[0])


def test_infeasible_problem_never_claims_convergence(torch):
    """Reference tests/test_regression_chambolle_pock.py:140-153."""
    from purin_amd import ChambollePockConfig, Projection, SolveStatus, prepare_projection

    p = Projection()
    y = p.add_variable(["u"])
    p.objective = 0.0
    p.constraints.add(y.u <= 0, y.u >= 1)
    layer = prepare_projection(p, method="chambolle-pock",
                               config=ChambollePockConfig(max_iterations=100), batch_size=1)
    out = layer.solve(torch.zeros((1, 1), dtype=torch.float64))
    assert int(out.status[0]) == int(SolveStatus.MAX_ITERATIONS)
    assert not bool(out.gradient_eligible[0])


def test_scaled_constraints_report_original_units(torch):
    """Reference tests/test_regression_chambolle_pock.py:156-164."""
    from purin_amd import Projection, prepare_projection

    p = Projection()
    y = p.add_variable(["u", "v"])
    p.objective = 0.0
    p.constraints.add(1000 * y.u + 1000 * y.v == 1000, y.u >= 0)
    layer = prepare_projection(p, method="chambolle-pock", batch_size=1)
    out = layer.solve(torch.tensor([[2.0, 0.0]], dtype=torch.float64))
    assert bool(out.gradient_eligible[0])
    assert abs(float(out.y.sum()) * 1000 - 1000) <= layer.config.tolerance


def test_tied_scaled_bounds_restore_duals_and_slacks(torch):
    """Reference tests/test_regression_cp_bound_presolve.py:13-27."""
    from purin_amd import Projection, SolveStatus, prepare_projection

    p = Projection()
    y = p.add_variable(["u", "v"])
    p.objective = 0.0
    p.constraints.add(y.u >= 0, 2 * y.u >= 0, y.u <= 2, y.v <= 1)
    layer = prepare_projection(p, method="chambolle-pock", batch_size=1)
    out = layer.solve(torch.tensor([[-3.0, 4.0]], dtype=torch.float64))
    np.testing.assert_allclose(out.y.detach().cpu(), [[0.0, 1.0]], atol=1e-10)
    np.testing.assert_allclose(out.multipliers_ineq.cpu(), [[1.5, 0.75, 0.0, 3.0]], atol=1e-9)
    np.testing.assert_allclose(out.slacks.cpu(), [[0.0, 0.0, 2.0, 0.0]], atol=1e-10)
    assert int(out.status[0]) == int(SolveStatus.CONVERGED)
    assert layer.plan.m == 0
    x = torch.tensor([[-3.0, 4.0]], dtype=torch.float64, device="cuda", requires_grad=True)
    layer(x).sum().backward()
    np.testing.assert_allclose(x.grad.cpu(), 0.0, atol=1e-9)


@pytest.mark.parametrize("seed", [12, 42])
def test_coupled_qp_matches_exact_projection_and_fd(torch, seed):
    """Reference tests/test_regression_cp_bound_presolve.py:56-109 (OSQP -> exact projection)."""
    from oracle import qp as bf
    from purin_amd import Projection, prepare_projection

    rng = np.random.default_rng(seed)
    p = Projection()
    y = p.add_variable(["u", "v", "w"])
    p.objective = 0.0
    p.constraints.add(y.u + y.v + y.w == 1, y.u >= 0, y.v >= -0.5, y.w <= 0.7,
                      2 * y.u - y.v <= 0.9)
    layer = prepare_projection(p, method="chambolle-pock", batch_size=1)
    x = rng.normal(size=(1, 3))
    matrix = np.array([[1.0, 1.0, 1.0], [-1.0, 0.0, 0.0], [0.0, -1.0, 0.0], [0.0, 0.0, 1.0],
                       [2.0, -1.0, 0.0]])
    upper = np.array([1.0, 0.0, 0.5, 0.7, 0.9])
    ref = bf.project_bruteforce(x[0], matrix[:1], upper[:1], matrix[1:], upper[1:])[0]
    out = layer.solve(torch.as_tensor(x))
    np.testing.assert_allclose(out.y[0].detach().cpu(), ref, atol=2e-8)
    mult = np.r_[out.multipliers_eq[0].cpu().numpy(), out.multipliers_ineq[0].cpu().numpy()]
    np.testing.assert_allclose((out.y[0].detach().cpu().numpy() - x[0]) + matrix.T @ mult, 0.0,
                               atol=1e-9)
    assert bool(out.gradient_eligible[0])
    g = torch.as_tensor(rng.normal(size=(1, 3)), device="cuda")
    xt = torch.as_tensor(x, device="cuda").requires_grad_(True)
    (layer(xt) * g).sum().backward()
    for i in range(3):
        d = np.zeros_like(x)
        d[0, i] = 1e-4
        fd = float(((layer(torch.as_tensor(x + d)) - layer(torch.as_tensor(x - d))) * g).sum()) / 2e-4
        np.testing.assert_allclose(float(xt.grad[0, i]), fd, atol=2e-5)


def make_problem(inequalities=False):
    from purin_amd import Projection

    problem = Projection()
    pb = problem.add_parameter(["b"])
    y = problem.add_variable(["u", "v"])
    problem.objective = 0.0
    problem.constraints.add(y.u + y.v == pb.b)
    if inequalities:
        problem.constraints.add(y.u >= 0)
        problem.constraints.add(y.v >= 0)
    return problem


@pytest.mark.parametrize("dtype,atol", [("float64", 2e-6), ("float32", 5e-5)])
def test_affine_projection_and_analytic_jacobian(torch, dtype, atol):
    """Reference tests/test_projections.py:65-75 and .github/scripts/numerical_regression.py:23-82
    (fp32 uses that script's settings: tolerance 1e-6, adjoint/inexact tolerance 1e-5,
    linear-solver tolerance 1e-6)."""
    from dataclasses import replace

    from purin_amd import ChambollePockConfig, Distance, ImplicitGradientConfig, LinearSolverConfig

    cfg = ChambollePockConfig(max_iterations=3000, tolerance=1e-6 if dtype == "float32" else 1e-10)
    if dtype == "float32":
        cfg = replace(cfg, implicit_gradient=ImplicitGradientConfig(adjoint_tolerance=1e-5,
                                                                    inexact_tolerance=1e-5),
                      linear_solver=LinearSolverConfig(tolerance=1e-6))
    project = Distance(make_problem(), "chambolle-pock", cfg).prepare(batch_size=1, dtype=dtype)
    tdt = torch.float64 if dtype == "float64" else torch.float32
    target = torch.tensor([[0.8, 0.7]], dtype=tdt, device="cuda")
    context = torch.ones((1, 1), dtype=tdt)
    np.testing.assert_allclose(project(target, context).detach().cpu(), [[0.55, 0.45]], atol=atol)
    d = jac(torch, lambda x: project(x[None, :], context)[0], target[0])
    np.testing.assert_allclose(d, [[0.5, -0.5], [-0.5, 0.5]], atol=atol)


@pytest.mark.parametrize("accelerated", [False, True])
def test_cp_variants_with_active_inequality(torch, accelerated):
    """Reference tests/test_projections.py:78-97."""
    from purin_amd import ChambollePockConfig, Distance

    cfg = ChambollePockConfig(accelerated=accelerated, tolerance=1e-9, max_iterations=3000)
    project = Distance(make_problem(inequalities=True), "chambolle-pock", cfg).prepare(batch_size=1)
    np.testing.assert_allclose(
        project(torch.tensor([[2.0, -1.0]], dtype=torch.float64),
                torch.ones((1, 1), dtype=torch.float64)).detach().cpu(), [[1.0, 0.0]], atol=2e-6)


def test_weighted_projection_protocol_and_gradient(torch):
    """Reference tests/test_projections.py:121-124, tests/test_training_metric_contracts.py:63-83."""
    from purin_amd import WeightedDistance

    prepared = WeightedDistance(make_problem(), [1.0, 4.0], method="chambolle-pock").prepare(
        batch_size=1)
    target = torch.tensor([[2.0, 0.0]], dtype=torch.float64, device="cuda")
    context = torch.ones((1, 1), dtype=torch.float64)
    expected = [[1.2, -0.2]]
    with pytest.raises(ValueError, match="warm starts"):
        prepared.solve(target, context, initial_state=torch.tensor([[1.2, -0.2]]))
    np.testing.assert_allclose(prepared.solve(target, context).y.detach().cpu(), expected, atol=2e-5)
    np.testing.assert_allclose(prepared.project_training(target, context).y_tilde.detach().cpu(),
                               expected, atol=2e-5)
    np.testing.assert_allclose(prepared.with_info(target, context)[0].detach().cpu(), expected,
                               atol=2e-5)
    d = jac(torch, lambda x: prepared(x[None], context)[0], target[0])
    np.testing.assert_allclose(d, [[0.2, -0.8], [-0.2, 0.8]], atol=2e-5)


@pytest.mark.parametrize("diagonal", [False, True])
def test_parameter_dependent_sparse_coefficients(torch, diagonal):
    """Reference tests/test_regression_chambolle_pock.py:116-137 and
    tests/test_regression_cp_diagonal_steps.py:83-112: ``a u + v == 1``; y and
    dy/da through torch autograd (purin_cp_project_values / adjoint_values)."""
    from purin_amd import (ChambollePockConfig, ImplicitGradientConfig, Projection,
                           prepare_projection)

    p = Projection()
    t = p.add_parameter(["a"])
    y = p.add_variable(["u", "v"])
    p.objective = 0.0
    p.constraints.add(t.a * y.u + y.v == 1)
    cfg = ChambollePockConfig(
        diagonal_preconditioning=diagonal,
        implicit_gradient=ImplicitGradientConfig(differentiate_problem_parameters=True))
    layer = prepare_projection(p, method="chambolle-pock", config=cfg, batch_size=1)
    x = torch.tensor([[0.2, 0.3]], dtype=torch.float64, device="cuda")
    theta = torch.tensor([[2.0]], dtype=torch.float64, device="cuda")

    def expected(t):
        a = t[0, 0]
        return x - torch.stack([a, torch.ones_like(a)])[None] * (a * 0.2 + 0.3 - 1) / (a * a + 1)

    np.testing.assert_allclose(layer(x, theta).detach().cpu(), expected(theta).cpu(), atol=1e-8)
    np.testing.assert_allclose(jac(torch, lambda t: layer(x, t), theta),
                               jac(torch, expected, theta), atol=2e-7)


def test_parameter_dependent_bound_sign_zero_and_derivative(torch):
    """Reference tests/test_regression_cp_bound_presolve.py:30-53: ``a u <= b``."""
    from purin_amd import (ChambollePockConfig, ImplicitGradientConfig, Projection,
                           prepare_projection)

    p = Projection()
    t = p.add_parameter(["a", "b"])
    y = p.add_variable(["u"])
    p.objective = 0.0
    p.constraints.add(t.a * y.u <= t.b)
    cfg = ChambollePockConfig(
        implicit_gradient=ImplicitGradientConfig(differentiate_problem_parameters=True))
    layer = prepare_projection(p, method="chambolle-pock", config=cfg, batch_size=1)
    f64 = dict(dtype=torch.float64, device="cuda")
    x = torch.tensor([[3.0]], **f64)
    theta = torch.tensor([[2.0, 1.0]], **f64)
    np.testing.assert_allclose(layer(x, theta).detach().cpu(), [[0.5]], atol=1e-10)
    j = jac(torch, lambda z: layer(x, z), theta)
    np.testing.assert_allclose(j[0, 0, 0], [-0.25, 0.5], atol=1e-8)
    np.testing.assert_allclose(
        layer(torch.tensor([[-3.0]], **f64), torch.tensor([[-2.0, 1.0]], **f64)).detach().cpu(),
        [[-0.5]], atol=1e-10)
    out = layer.solve(x, torch.tensor([[0.0, -1.0]], **f64))
    assert not bool(out.gradient_eligible[0])
    xg = x.clone().requires_grad_(True)
    layer(xg, torch.tensor([[0.0, -1.0]], **f64)).sum().backward()
    np.testing.assert_allclose(xg.grad.cpu(), 0.0)
    np.testing.assert_allclose(layer(x, torch.tensor([[0.0, 1.0]], **f64)).detach().cpu(),
                               x.cpu())


def test_products_of_parameters_are_reported_unsupported(torch):
    from purin_amd import Projection, prepare_projection

    p = Projection()
    t = p.add_parameter(["a"])
    y = p.add_variable(["u", "v"])
    p.constraints.add(y.u + y.v == t.a * t.a)
    with pytest.raises(NotImplementedError, match="affine in the parameters"):
        prepare_projection(p, method="chambolle-pock", batch_size=1)


@pytest.mark.parametrize("early_stop", [False, True])
def test_front_end_runs_the_resident_kernel_with_shared_bounds(torch, early_stop):
    """A config2-shaped problem through the PURIN API: its bound rows are
    constant, so the front end passes shared_bounds and the call runs the
    resident kernel; the result (y, multipliers, statuses, iterations,
    residuals, the VJP) is bit-identical to the per-sample-bounds call."""
    import scipy.sparse as sp

    from purin_amd import ChambollePockConfig, Distance
    from purin_amd import workloads

    w = workloads.small_random(31, n=900, me=120, mi=300, width=6, batch=70, accelerated=True,
                               target_sd=0.2)
    me, M = w.me, w.rows_total
    A = sp.csr_matrix((w.data, w.indices, w.indptr), shape=(M, w.n))
    from purin_amd import MatrixProblem

    pa_problem = MatrixProblem(
        P=sp.identity(w.n, format="csr"), q0=np.zeros(w.n), A_eq=A[:me], b_eq0=w.rhs[:me],
        A_ineq=A[me:], b_ineq0=w.rhs[me:])
    cfg = ChambollePockConfig(accelerated=True, max_iterations=500, early_stop=early_stop,
                              tolerance=1e-3)
    layer = Distance(pa_problem, config=cfg).prepare(batch_size=w.batch)
    assert layer.shared_bounds
    y_hat = torch.as_tensor(w.target, device="cuda").requires_grad_(True)
    out = layer.solve(y_hat)
    cot = torch.as_tensor(np.random.default_rng(3).normal(size=w.target.shape), device="cuda")
    (g_api,) = torch.autograd.grad(out.y, y_hat, cot)
    plan = layer.plan
    rhs = torch.as_tensor(np.tile(w.rhs, (w.batch, 1)), device="cuda")
    kw = dict(max_iterations=500, early_stop=early_stop, tolerance=1e-3)
    shared = plan.project(y_hat.detach(), rhs, shared_bounds=True, timing=True, save=True, **kw)
    assert plan.last_timing()["resident"] == 1
    per = plan.project(y_hat.detach(), rhs, shared_bounds=False, timing=True, save=True, **kw)
    assert plan.last_timing()["resident"] == 1
    if early_stop:  # the stop test fired for some samples (about 380-530 iterations)
        assert np.any(per.iterations.cpu().numpy() < 500)
    for a, b in ((out.y, shared.y), (shared.y, per.y), (shared.multipliers, per.multipliers),
                 (shared.status, per.status), (shared.iterations, per.iterations),
                 (shared.residual, per.residual), (shared.eligible, per.eligible)):
        assert torch.equal(a.detach(), b)
    ga = plan.adjoint(shared.saved, None, None, cot, force_eligible=True)
    gb = plan.adjoint(per.saved, None, None, cot, force_eligible=True)
    assert torch.equal(ga.g_target, gb.g_target) and torch.equal(ga.g_rhs, gb.g_rhs)
    eligible = shared.eligible.bool()
    assert torch.equal(g_api[eligible], plan.adjoint(shared.saved, None, None, cot).g_target[eligible])


def test_front_end_per_sample_bounds_when_a_bound_row_moves(torch):
    """``u >= b`` with b a parameter: the bound rows differ per sample, so the
    front end keeps per-sample bounds, and each sample gets its own bound."""
    from purin_amd import ChambollePockConfig, Projection, prepare_projection

    p = Projection()
    t = p.add_parameter(["b"])
    y = p.add_variable(["u", "v"])
    p.constraints.add(y.u + y.v == 1, y.u >= t.b)
    layer = prepare_projection(p, config=ChambollePockConfig(), batch_size=2)
    assert not layer.shared_bounds
    out = layer.solve(torch.tensor([[0.0, 0.0], [0.0, 0.0]], dtype=torch.float64, device="cuda"),
                      torch.tensor([[0.2], [0.8]], dtype=torch.float64, device="cuda"))
    np.testing.assert_allclose(out.y.cpu().numpy(), [[0.5, 0.5], [0.8, 0.2]], atol=1e-8)
