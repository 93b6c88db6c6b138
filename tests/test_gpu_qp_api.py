"""The reference's diagonal-QP tests through this build's front end
(purin_amd/diagonal_qp.py) on the GPU; gradients use torch autograd, whose
backward is purin_cp_qp_adjoint."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as _torch

    if not _torch.cuda.is_available():
        pytest.skip("needs a GPU")
    return _torch


@pytest.mark.parametrize("accelerated", [False, True])
@pytest.mark.parametrize("scaling", [False, True])
def test_diagonal_qp_value_and_coefficient_gradient(torch, accelerated, scaling):
    """Reference tests/test_diagonal_qp.py:13-48."""
    from purin_amd import ChambollePockConfig
    from purin_amd.diagonal_qp import dense_qp_data

    f64 = dict(dtype=torch.float64, device="cuda")
    structure, data = dense_qp_data(
        torch.tensor([[2.0, 4.0]], **f64), torch.tensor([[-2.0, -4.0]], **f64),
        torch.ones((1, 1, 2), **f64), torch.tensor([1.0], **f64), torch.empty((0, 2), **f64),
        torch.empty(0, **f64), -np.inf, np.inf)
    config = ChambollePockConfig(accelerated=accelerated, row_scaling=scaling, tolerance=1e-9,
                                 max_iterations=3000)
    solver = structure.prepare(batch_size=1, config=config)
    result = solver.solve(data)
    np.testing.assert_allclose(result.y.detach().cpu(), [[1 / 3, 2 / 3]], atol=1e-8)
    assert float(result.residual_inf_norm[0]) < 1e-8
    expected = -np.diag([0.5, 0.25]) + np.outer([0.5, 0.25], [0.5, 0.25]) / 0.75
    actual = torch.autograd.functional.jacobian(
        lambda c: solver.solve(data._replace(c=c[None, :])).y[0], data.c[0])
    np.testing.assert_allclose(actual.cpu(), expected, atol=1e-7)
    warm = solver.solve(data, initial_y=result.y, initial_dual=result.multipliers_eq)
    np.testing.assert_allclose(warm.y.detach().cpu(), result.y.detach().cpu(), atol=1e-8)
    with pytest.raises(ValueError):
        solver.solve(data._replace(q=torch.ones((2, 2), **f64)))
    with pytest.raises(ValueError):
        solver.solve(data, initial_y=torch.zeros((2, 2), **f64))
    with pytest.raises(ValueError):
        solver.solve(data, initial_dual=torch.zeros((2, 1), **f64))


def test_every_input_is_differentiable(torch):
    """Gradients w.r.t. q, c, values, rhs, lower and upper, and through the
    multipliers, against central differences of the forward (one active bound,
    one equality, one inequality)."""
    from purin_amd import ChambollePockConfig
    from purin_amd.diagonal_qp import QPData, QPStructure

    f64 = dict(dtype=torch.float64, device="cuda")
    structure = QPStructure(3, ((0, 1, 2),), ((0, 2),))
    cfg = ChambollePockConfig(tolerance=1e-12, max_iterations=100000)
    solver = structure.prepare(batch_size=1, config=cfg)
    base = QPData(torch.tensor([[1.0, 2.0, 1.5]], **f64), torch.tensor([[-1.0, 0.5, -2.0]], **f64),
                  torch.tensor([[[1.0, 1.0, 1.0], [1.0, 2.0, 0.0]]], **f64),
                  torch.tensor([[1.0, 0.8]], **f64), torch.tensor([[-1.0, -0.1, -1.0]], **f64),
                  torch.tensor([[1.0, 1.0, 1.0]], **f64))
    w_y = torch.tensor([[0.3, -1.2, 0.7]], **f64)
    w_m = torch.tensor([[0.5, -0.4]], **f64)

    def f(*xs):
        r = solver.solve(QPData(*xs))
        return (r.y * w_y).sum() + (torch.cat((r.multipliers_eq, r.multipliers_ineq), 1)
                                    * w_m).sum()

    inputs = [x.clone().requires_grad_(True) for x in base]
    r = solver.solve(QPData(*inputs))
    assert int(r.status[0]) == 0
    f(*inputs).backward()
    h = 1e-6
    for k, x in enumerate(base):
        flat = x.reshape(-1)
        for j in range(flat.numel()):
            if k == 2 and j == 5:  # padding slot of the second row: no coefficient
                continue
            up = [t.clone() for t in base]
            dn = [t.clone() for t in base]
            up[k].reshape(-1)[j] += h
            dn[k].reshape(-1)[j] -= h
            want = float((f(*up) - f(*dn)) / (2 * h))
            got = float(inputs[k].grad.reshape(-1)[j])
            assert abs(got - want) <= 2e-6, (k, j, got, want)


def test_local_quadratic_training_protocol(torch):
    """Reference tests/test_diagonal_qp.py:53-106: the prepared local QP solves to
    [1/3, 2/3] through solve, __call__, with_info and project_training."""
    import purin_amd as pa
    from tests.test_frontend import _local_problem

    definition = pa.LocalQuadratic(
        _local_problem(), lower=lambda p: torch.zeros(2, dtype=p.dtype, device=p.device),
        upper=2.0, config=pa.ChambollePockConfig(tolerance=1e-9, max_iterations=3000))
    f64 = dict(dtype=torch.float64, device="cuda")
    context = torch.ones((1, 1), **f64)
    anchor = torch.tensor([[0.4, 0.5]], **f64)
    prepared = definition.prepare(batch_size=1)
    result = prepared.solve(anchor, context)
    np.testing.assert_allclose(result.y.detach().cpu(), [[1 / 3, 2 / 3]], atol=1e-8)
    np.testing.assert_allclose(prepared(anchor, context).detach().cpu(),
                               result.y.detach().cpu(), atol=1e-8)
    np.testing.assert_allclose(prepared.with_info(anchor, context)[0].detach().cpu(),
                               result.y.detach().cpu(), atol=1e-8)
    for kwargs in [{}, {"multipliers_eq": result.multipliers_eq,
                        "multipliers_ineq": result.multipliers_ineq}]:
        np.testing.assert_allclose(
            prepared.project_training(anchor, context, **kwargs).y_tilde.detach().cpu(),
            result.y.detach().cpu(), atol=1e-8)
    # the context (the equality's rhs) is differentiable through the local QP:
    # y = argmin over u + v = p of the quadratic; dy/dp = Q^-1 1 / (1'Q^-1 1) = [2/3, 1/3]
    ctx = context.clone().requires_grad_(True)
    jac = torch.autograd.functional.jacobian(lambda p: prepared(anchor, p)[0], ctx)
    np.testing.assert_allclose(jac.reshape(2).cpu(), [2 / 3, 1 / 3], atol=1e-7)


@pytest.mark.parametrize("accelerated", [False, True])
@pytest.mark.parametrize("equilibrate", [False, True])
def test_dense_cp_matches_analytic_equality_qp(torch, accelerated, equilibrate):
    """Reference tests/test_dense_cp.py:20-49 through purin_amd.dense (the
    derivative through the equilibration by torch autograd)."""
    from purin_amd.dense import solve_dense_implicit

    f64 = dict(dtype=torch.float64, device="cuda")
    q = torch.tensor([[2.0, 4.0]], **f64)
    c = torch.tensor([[-2.0, -4.0]], **f64)
    A = torch.ones((1, 1, 2), **f64)
    b = torch.ones((1, 1), **f64)
    C = torch.tensor([[[-1.0, 0.0]]], **f64)
    d = torch.zeros((1, 1), **f64)
    lo = torch.zeros((1, 2), **f64)
    hi = torch.ones((1, 2), **f64) * 2
    kw = dict(accelerated=accelerated, equilibrate=equilibrate, tolerance=1e-13,
              max_iterations=20000)
    actual = solve_dense_implicit(q, c, A, b, C, d, lo, hi, **kw)
    np.testing.assert_allclose(actual[0].detach().cpu(), [[1 / 3, 2 / 3]], atol=1e-6)
    warm = solve_dense_implicit(q, c, A, b, C, d, lo, hi, y0=actual[0], lambda0=actual[1],
                                mu0=actual[2], **kw)
    np.testing.assert_allclose(warm[0].detach().cpu(), actual[0].detach().cpu(), atol=1e-6)
    derivative = torch.autograd.functional.jacobian(
        lambda lin: solve_dense_implicit(q, lin, A, b, C, d, lo, hi, **kw)[0], c)
    expected = -np.diag([0.5, 0.25]) + np.outer([0.5, 0.25], [0.5, 0.25]) / 0.75
    np.testing.assert_allclose(derivative[0, :, 0, :].cpu(), expected, atol=1e-6)


def test_dense_empty_constraints(torch):
    """Reference tests/test_dense_cp.py:52-73."""
    from purin_amd.dense import solve_dense_implicit

    f64 = dict(dtype=torch.float64, device="cuda")
    y = solve_dense_implicit(torch.ones((1, 2), **f64), torch.tensor([[-1.0, -2.0]], **f64),
                             torch.zeros((1, 0, 2), **f64), torch.zeros((1, 0), **f64),
                             torch.zeros((1, 0, 2), **f64), torch.zeros((1, 0), **f64),
                             torch.zeros((1, 2), **f64), torch.ones((1, 2), **f64) * 3,
                             equilibrate=True, tolerance=1e-14)[0]
    np.testing.assert_allclose(y.cpu(), [[1.0, 2.0]], atol=1e-6)


def test_dense_packed_support_and_gradients(torch):
    """inequality_support (sparse_layer.py:44-122) gives the same solution as the
    dense rows with those entries; gradients against central differences."""
    from purin_amd.dense import solve_dense_implicit

    f64 = dict(dtype=torch.float64, device="cuda")
    rng = np.random.default_rng(8)
    n = 4
    q = torch.tensor(rng.uniform(1, 2, (1, n)), **f64)
    c = torch.tensor(rng.normal(size=(1, n)), **f64)
    A = torch.tensor(rng.normal(size=(1, 1, n)), **f64)
    b = torch.tensor([[0.2]], **f64)
    support = ((0, 2), (1, 3))
    C = torch.zeros((1, 2, n), **f64)
    C[0, 0, [0, 2]] = torch.tensor([1.0, -0.5], **f64)
    C[0, 1, [1, 3]] = torch.tensor([0.7, 1.2], **f64)
    d = torch.tensor([[0.1, 0.05]], **f64)
    lo, hi = -torch.ones((1, n), **f64), torch.ones((1, n), **f64)
    kw = dict(tolerance=1e-12, max_iterations=50000, adjoint_iterations=500)
    dense = solve_dense_implicit(q, c, A, b, C, d, lo, hi, **kw)
    packed = solve_dense_implicit(q, c, A, b, C, d, lo, hi, inequality_support=support, **kw)
    np.testing.assert_allclose(packed[0].detach().cpu(), dense[0].detach().cpu(), atol=1e-9)
    w = torch.tensor(rng.normal(size=(1, n)), **f64)
    cc = c.clone().requires_grad_(True)
    dd = d.clone().requires_grad_(True)
    (solve_dense_implicit(q, cc, A, b, C, dd, lo, hi, inequality_support=support, **kw)[0]
     * w).sum().backward()
    h = 1e-6
    for x, g in ((c, cc.grad), (d, dd.grad)):
        for j in range(x.shape[1]):
            up, dn = x.clone(), x.clone()
            up[0, j] += h
            dn[0, j] -= h
            args_up = (up, d) if x is c else (c, up)
            args_dn = (dn, d) if x is c else (c, dn)
            f = lambda cv, dv: float((solve_dense_implicit(q, cv, A, b, C, dv, lo, hi,
                                                           inequality_support=support, **kw)[0]
                                      * w).sum())
            want = (f(*args_up) - f(*args_dn)) / (2 * h)
            assert abs(float(g[0, j]) - want) <= 1e-5, (j, float(g[0, j]), want)
