"""GPU parity of the dense CP adapter's forward (purin_cp_dense_solve) with the
oracle (oracle/dense.py: solve_dense, chambolle_pock/dense.py:26-105 -- factored
prox, no freezing, no stationarity test, power-iteration steps), through the C
ABI.  The oracle is pinned in tests/test_oracle_dense.py."""

import numpy as np
import pytest

from oracle import dense as od
from tests._gpu import rel_err, require_gpu, to_np

pytestmark = pytest.mark.gpu

TOL = {np.float64: 1e-10, np.float32: 1e-4}


def _dense_plan(n, me, mi, dtype, support=None, **kw):
    import torch
    from purin_amd.plan import Plan

    rows = [list(range(n))] * me + ([list(range(n))] * mi if support is None else
                                    [sorted(r) for r in support])
    indptr = np.zeros(len(rows) + 1, np.int64)
    indptr[1:] = np.cumsum([len(r) for r in rows])
    indices = np.asarray([c for r in rows for c in r], np.int32)
    return Plan(n, me, mi, indptr, indices, np.ones(indptr[-1]),
                dtype=torch.float64 if dtype == np.float64 else torch.float32,
                bound_presolve=False, row_scaling=False, norm_bound=False, device="cuda", **kw)


def _problem(seed, B=24, n=12, me=3, mi=5):
    rng = np.random.default_rng(seed)
    q = rng.uniform(0.5, 3.0, (B, n))
    c = rng.normal(size=(B, n))
    A = rng.normal(size=(B, me, n))
    C = rng.normal(size=(B, mi, n))
    x0 = rng.uniform(-0.3, 0.3, (B, n))
    b = np.einsum("bmn,bn->bm", A, x0)
    d = np.einsum("bmn,bn->bm", C, x0) + rng.uniform(0.1, 0.5, (B, mi))
    lo, hi = np.full((B, n), -1.0), np.full((B, n), 1.0)
    return q, c, A, b, C, d, lo, hi


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("accelerated", [False, True])
@pytest.mark.parametrize("early_stop", [False, True])
def test_dense_solve_matches_oracle(dtype, accelerated, early_stop):
    require_gpu()
    q, c, A, b, C, d, lo, hi = (x.astype(dtype) for x in _problem(51))
    B, n = q.shape
    me, mi = A.shape[1], C.shape[1]
    iters = 400
    tol = (1e-7 if dtype == np.float64 else 1e-3) if early_stop else 0.0
    y, lam, mu, it, _ = od.solve_dense(q, c, A, b, C, d, lo, hi, accelerated=accelerated,
                                       max_iterations=iters, tolerance=max(tol, 1e-300))
    plan = _dense_plan(n, me, mi, dtype, accelerated=accelerated)
    values = np.concatenate((A, C), axis=1).reshape(B, -1)
    gy, gm, git, _ = plan.dense_solve(q, c, np.concatenate((b, d), axis=1), lo, hi, values=values,
                                      tolerance=max(tol, 1e-30), max_iterations=iters,
                                      early_stop=early_stop, check_every=7)
    # no freezing: every sample runs until the last one is accepted
    np.testing.assert_array_equal(to_np(git), it)
    assert len(np.unique(it)) == 1
    if early_stop and dtype == np.float64 and not accelerated:
        assert it[0] < iters  # the stop test fired (accelerated fp64 stalls above 1e-7)
    assert rel_err(to_np(gy), y) <= TOL[dtype]
    assert rel_err(to_np(gm), np.concatenate((lam, mu), axis=1)) <= TOL[dtype]


def test_dense_packed_inequality_support():
    """A packed inequality support (sparse_layer.py:44-122): the inequality rows
    keep only their listed columns; the same iteration otherwise."""
    require_gpu()
    q, c, A, b, C, d, lo, hi = _problem(52, B=16, n=10, me=2, mi=4)
    support = [[0, 3, 4], [1, 2], [5, 6, 7, 9], [8]]
    mask = np.zeros(C.shape[1:], bool)
    for i, r in enumerate(support):
        mask[i, r] = True
    C = np.where(mask[None], C, 0.0)
    x0 = np.zeros((16, 10))
    d = np.abs(d)
    y, lam, mu, it, _ = od.solve_dense(q, c, A, b, C, d, lo, hi, max_iterations=300,
                                       tolerance=1e-300)
    plan = _dense_plan(10, 2, 4, np.float64, support=support)
    packed = np.concatenate((A.reshape(16, -1), C[:, mask]), axis=1)
    gy, gm, git, _ = plan.dense_solve(q, c, np.concatenate((b, d), axis=1), lo, hi,
                                      values=packed, max_iterations=300, early_stop=False)
    assert rel_err(to_np(gy), y) <= 1e-10
    assert rel_err(to_np(gm), np.concatenate((lam, mu), axis=1)) <= 1e-9


def test_dense_known_answer_and_warm_start():
    """Reference tests/test_dense_cp.py:20-45: [1/3, 2/3] and warm start."""
    require_gpu()
    plan = _dense_plan(2, 1, 1, np.float64)
    q, c = np.array([[2.0, 4.0]]), np.array([[-2.0, -4.0]])
    vals = np.array([[1.0, 1.0, -1.0, 0.0]])
    rhs = np.array([[1.0, 0.0]])
    lo, hi = np.zeros((1, 2)), np.full((1, 2), 2.0)
    for accelerated in (False, True):
        plan = _dense_plan(2, 1, 1, np.float64, accelerated=accelerated)
        y, m, it, _ = plan.dense_solve(q, c, rhs, lo, hi, values=vals, tolerance=1e-13,
                                       max_iterations=20000)
        np.testing.assert_allclose(to_np(y), [[1 / 3, 2 / 3]], atol=1e-6)
        w, _, _, _ = plan.dense_solve(q, c, rhs, lo, hi, values=vals, y0=y, dual0=m,
                                      tolerance=1e-13, max_iterations=20000)
        np.testing.assert_allclose(to_np(w), to_np(y), atol=1e-6)


@pytest.mark.parametrize("with_dual_cotangent", [False, True])
@pytest.mark.parametrize("tol,iters,bar", [(1e-6, 50, 1e-5), (1e-12, 400, 1e-9)])
def test_dense_adjoint_matches_oracle_at_the_same_state(with_dual_cotangent, tol, iters, bar):
    """BiCGSTAB over the batch with the frozen prox (dense_implicit.py:160-210) at
    the GPU's state, with the same iteration count.  Converged (1e-12) the
    gradients agree to 1e-9; at the reference's 1e-6 the unconverged iterate
    depends on the rounding of the global dot products (summed in another
    order), and agrees to 10 x that tolerance.  The iteration counts agree to
    two (the last stop test moves with the operator's rounding)."""
    require_gpu()
    q, c, A, b, C, d, lo, hi = _problem(53, B=8, n=10, me=2, mi=4)
    B, n = q.shape
    me, mi = 2, 4
    plan = _dense_plan(n, me, mi, np.float64)
    values = np.concatenate((A, C), axis=1)
    rhs = np.concatenate((b, d), axis=1)
    y, m, it, saved = plan.dense_solve(q, c, rhs, lo, hi, values=values.reshape(B, -1),
                                       tolerance=1e-10, max_iterations=20000, save=True)
    rng = np.random.default_rng(4)
    cot = rng.normal(size=(B, n))
    cotd = rng.normal(size=(B, me + mi)) if with_dual_cotangent else np.zeros((B, me + mi))
    want = od.implicit_vjp(q, c, values, rhs, lo, hi, me, to_np(y), to_np(m), cot, cotd,
                           tolerance=tol, adjoint_iterations=iters)
    got = plan.dense_adjoint(saved, q, c, cot, values=values.reshape(B, -1),
                             cot_dual=cotd if with_dual_cotangent else None, tolerance=tol,
                             max_iterations=iters)
    stats = plan.last_adjoint_stats()
    # the first iteration under the stop threshold moves with the operator's
    # rounding: with unit-roundoff noise on each operator output the oracle's
    # own count spans 59-61 here (10 noise seeds, tolerance 1e-12)
    assert abs(stats["arnoldi_steps"] - want[5]) <= 2 and want[5] > 0
    np.testing.assert_array_equal(to_np(got.g_q), 0.0)
    for name, w in (("g_c", want[0]), ("g_values", want[1].reshape(B, -1)), ("g_rhs", want[2]),
                    ("g_lower", want[3]), ("g_upper", want[4])):
        assert rel_err(to_np(getattr(got, name)), w) <= bar, name
