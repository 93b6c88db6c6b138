"""Host-side front end: canonical rows, sign conventions, configuration validation.

CPU only (no kernel is launched).
"""

import math

import numpy as np
import pytest

import purin_amd as pa
from purin_amd.problems import CanonicalRows


def test_public_names_match_the_reference_cp_surface():
    for name in ("Projection", "ParametricQP", "MatrixProblem", "ChambollePockConfig",
                 "LinearSolverConfig", "ImplicitGradientConfig", "SolveStatus",
                 "prepare_projection", "registered_methods", "Distance", "WeightedDistance"):
        assert getattr(pa, name) is not None
    assert pa.registered_methods() == ("chambolle-pock",)
    assert [int(s) for s in pa.SolveStatus] == [0, 1, 2, 3, 4]


def test_symbolic_rows_signs_and_rhs_map():
    """``u + v == b`` and ``u >= 0``: expressions.py:298-309 sign convention."""
    p = pa.Projection()
    t = p.add_parameter(["b"])
    y = p.add_variable(["u", "v"])
    p.objective = 0.0
    p.constraints.add(y.u + y.v == t.b, y.u >= 0, 2 * y.v <= 3 - t.b)
    c = p.canonicalize()
    assert (c.me, c.mi, c.n, c.parameter_size) == (1, 2, 2, 1)
    np.testing.assert_array_equal(c.indptr, [0, 2, 3, 4])
    np.testing.assert_array_equal(c.indices, [0, 1, 0, 1])
    np.testing.assert_array_equal(c.values, [1.0, 1.0, -1.0, 2.0])
    np.testing.assert_array_equal(c.rhs([[5.0]]), [[5.0, 0.0, -2.0]])
    assert c.affine and not c.parametric_coefficients


def test_nonlinear_and_parametric_coefficients_are_flagged():
    p = pa.Projection()
    y = p.add_variable(["u"])
    p.constraints.add(y.u ** 2 <= 1)
    assert not p.canonicalize().affine
    q = pa.Projection()
    a = q.add_parameter(["a"])
    z = q.add_variable(["u", "v"])
    q.constraints.add(a.a * z.u + z.v == 1)
    assert q.canonicalize().parametric_coefficients
    with pytest.raises(TypeError):
        bool(z.u <= 1)


def test_parameter_dependent_coefficients_form_an_affine_value_map():
    """``(2a + 1) u - b v <= 3 + b`` and ``a u >= 0``: per-entry values
    values0 + theta @ value_map.T in the CSR entry order; a structural entry
    whose constant part is zero stays in the row's support."""
    q = pa.Projection()
    t = q.add_parameter(["a", "b"])
    z = q.add_variable(["u", "v"])
    q.constraints.add((2 * t.a + 1) * z.u - t.b * z.v <= 3 + t.b, t.a * z.u >= 0)
    c = q.canonicalize()
    assert c.parametric_coefficients and c.parameter_affine and c.affine
    np.testing.assert_array_equal(c.indptr, [0, 2, 3])
    np.testing.assert_array_equal(c.indices, [0, 1, 0])
    np.testing.assert_array_equal(c.values, [1.0, 0.0, 0.0])
    np.testing.assert_array_equal(c.value_map, [[2.0, 0.0], [0.0, -1.0], [-1.0, 0.0]])
    np.testing.assert_allclose(c.coefficient_values([[0.5, 2.0]]), [[2.0, -2.0, -0.5]])
    np.testing.assert_allclose(c.rhs([[0.5, 2.0]]), [[5.0, 0.0]])
    r = pa.Projection()
    s = r.add_parameter(["a"])
    w = r.add_variable(["u"])
    r.constraints.add(w.u <= s.a * s.a)
    assert not r.canonicalize().parameter_affine


def test_duplicate_symbols_rejected():
    p = pa.Projection()
    p.add_variable(["u"])
    with pytest.raises(ValueError, match="Duplicate"):
        p.add_parameter(["u"])


def test_matrix_problem_from_bounds_row_order():
    """Upper rows then lower rows, equalities where lower == upper (qp.py:308-398)."""
    A = np.array([[1, 1, 1], [1, 0, 0], [0, 1, 0], [0, 0, 1], [2, -1, 0]], float)
    m = pa.MatrixProblem.from_bounds(P=np.eye(3), q0=np.zeros(3), A=A,
                                     lower0=[1, 0, -0.5, -np.inf, -np.inf],
                                     upper0=[1, np.inf, np.inf, 0.7, 0.9])
    c = m.canonicalize()
    assert (c.me, c.mi) == (1, 4)
    np.testing.assert_array_equal(c.rhs0, [1.0, 0.7, 0.9, 0.0, 0.5])
    np.testing.assert_array_equal(c.values, [1, 1, 1, 1, 2, -1, -1, -1])


def test_matrix_problem_sparse_and_dense_agree():
    import scipy.sparse as sp

    rng = np.random.default_rng(0)
    A = rng.normal(size=(4, 6)) * (rng.uniform(size=(4, 6)) < 0.5)
    dense = pa.ParametricQP(P=np.eye(6), q0=np.zeros(6), A_ineq=A, b_ineq0=np.ones(4)).canonicalize()
    sparse = pa.ParametricQP(P=np.eye(6), q0=np.zeros(6), A_ineq=sp.csr_matrix(A),
                             b_ineq0=np.ones(4)).canonicalize()
    for f in ("indptr", "indices", "values", "rhs0"):
        np.testing.assert_array_equal(getattr(dense, f), getattr(sparse, f))


@pytest.mark.parametrize("kwargs,match", [
    (dict(tolerance=0.0), "tolerance"),
    (dict(tolerance=math.inf), "tolerance"),
    (dict(max_iterations=0), "max_iterations"),
    (dict(max_iterations=1.5), "max_iterations"),
    (dict(safety=1.0), "safety"),
    (dict(norm_iterations=0), "norm_iterations"),
    (dict(metric_diagonal=(1.0, -1.0)), "metric_diagonal"),
])
def test_config_validation_messages(kwargs, match):
    """Reference src/purin/solvers/chambolle_pock/config.py:50-61."""
    with pytest.raises(ValueError, match=match):
        pa.ChambollePockConfig(**kwargs)


def test_linear_and_gradient_config_validation():
    with pytest.raises(ValueError):
        pa.LinearSolverConfig(restart=0)
    with pytest.raises(ValueError):
        pa.ImplicitGradientConfig(policy="bogus")
    assert pa.ChambollePockConfig().linear_solver.restart == 30


def test_cpu_backend_and_unknown_methods_are_rejected():
    from purin_amd.projection import resolve_device

    with pytest.raises(ValueError, match="cpu"):
        resolve_device("cpu")
    with pytest.raises(ValueError, match="Unknown projection method"):
        pa.ProjectionMethod.normalize("admm")


def test_canonical_rows_rhs_broadcast():
    c = CanonicalRows(2, 1, 0, 1, np.array([0, 2]), np.array([0, 1], np.int32), np.ones(2),
                      np.array([0.5]), np.array([[2.0]]))
    np.testing.assert_array_equal(c.rhs([[1.0], [2.0]]), [[2.5], [4.5]])


def test_invalid_qp_structures():
    """Reference tests/test_diagonal_qp.py:109-137 (the parts that need no GPU)."""
    from purin_amd.diagonal_qp import QPStructure, dense_qp_data

    for args in [(0,), (2, ((0, 0),)), (2, ((2,),)), (2, ((-1,),))]:
        with pytest.raises(ValueError):
            QPStructure(*args)
    structure = QPStructure(2)
    with pytest.raises(ValueError):
        structure.prepare(batch_size=0)
    with pytest.raises(ValueError):
        structure.prepare(batch_size=1,
                          config=pa.ChambollePockConfig(metric_diagonal=(1.0, 1.0)))
    with pytest.raises(ValueError):
        dense_qp_data(np.ones(2), np.ones(2), np.empty((0, 2)), [], np.empty((0, 2)), [], -1, 1)
    s = QPStructure(3, ((0, 2),), ((1,), (0, 1, 2)))
    assert s.rows == ((0, 2), (1,), (0, 1, 2))


def _local_problem():
    import torch

    return pa.FunctionalProblem(
        parameter_size=1, variable_size=2,
        objective=lambda p, y: 0.5 * torch.sum(torch.tensor([2.0, 4.0], dtype=y.dtype,
                                                            device=y.device)
                                               * (y - 1) ** 2),
        equalities=lambda p, y: torch.stack([torch.sum(y) - p[0]]), equality_size=1,
        inequalities=lambda p, y: torch.stack([-y[0]]), inequality_size=1)


def test_local_quadratic_coefficients():
    """Reference tests/test_diagonal_qp.py:53-76 (the builder, on the CPU)."""
    import torch

    definition = pa.LocalQuadratic(_local_problem(), lower=lambda p: torch.zeros(2), upper=2.0)
    compiled = definition.compile()
    context = torch.ones((1, 1), dtype=torch.float64)
    anchor = torch.tensor([[0.4, 0.5]], dtype=torch.float64)
    data = compiled.build(context, anchor)
    np.testing.assert_allclose(data.q, [[2.0, 4.0]])
    np.testing.assert_allclose(data.c, [[-2.0, -4.0]])
    np.testing.assert_allclose(data.rhs, [[1.0, 0.0]])
    np.testing.assert_allclose(data.lower, [[0.0, 0.0]])
    np.testing.assert_allclose(data.upper, [[2.0, 2.0]])
    for badcontext, badanchor in [(context[0], anchor), (context, anchor[0]),
                                  (torch.ones((2, 1)), anchor), (torch.ones((1, 2)), anchor),
                                  (context, torch.ones((1, 3)))]:
        with pytest.raises(ValueError):
            compiled.build(badcontext, badanchor)
    for kwargs in [dict(rho=0), dict(diagonal_floor=-1), dict(rho=np.inf)]:
        with pytest.raises(ValueError):
            pa.LocalQuadratic(_local_problem(), **kwargs)


def test_front_end_shares_bounds_only_when_every_bound_row_is_constant():
    """Singleton inequality rows are the presolved bounds (bounds.py:320-326);
    their thresholds rhs/coef (bounds.py:193-209) are the same for every sample
    when no bound row's rhs depends on theta and the coefficients are shared."""
    from purin_amd.projection import bounds_are_shared, constant_rows

    p = pa.Projection()
    t = p.add_parameter(["b"])
    y = p.add_variable(["u", "v"])
    p.constraints.add(y.u + y.v == t.b, y.u >= 0, 2 * y.v <= 3, y.u - y.v <= t.b)
    c = p.canonicalize()
    np.testing.assert_array_equal(constant_rows(c), [False, True, True, False])
    assert bounds_are_shared(c)          # the two-entry row may depend on theta
    q = pa.Projection()
    s = q.add_parameter(["b"])
    z = q.add_variable(["u", "v"])
    q.constraints.add(z.u + z.v == 1, z.u >= s.b)   # a bound row that moves with theta
    assert not bounds_are_shared(q.canonicalize())
    r = pa.Projection()
    a = r.add_parameter(["a"])
    x = r.add_variable(["u", "v"])
    r.constraints.add(a.a * x.u + x.v == 1, x.u >= 0)  # per-sample coefficients
    assert not bounds_are_shared(r.canonicalize())
    m = pa.MatrixProblem(P=np.eye(2), q0=np.zeros(2), A_ineq=np.array([[1.0, 0.0], [0.0, 2.0]]),
                         b_ineq0=np.ones(2), b_ineq_parameter_map=np.array([[0.0], [1.0]]))
    assert not bounds_are_shared(m.canonicalize())
    empty = pa.Projection()
    empty.add_variable(["u", "v"])
    assert bounds_are_shared(empty.canonicalize())  # no rows at all
    assert constant_rows(empty.canonicalize()).shape == (0,)
