"""GPU parity with per-sample coefficients (purin_cp_project_values /
purin_cp_adjoint_values): the reference's parameter-dependent values
(B, m_tot, w) of src/purin/solvers/chambolle_pock/bounds.py:192-236, with
per-sample row scales, bounds, norm bounds, step schedules and tolerances.

The oracle's per-sample path is pinned in tests/test_oracle_values.py (the
reference's known answers and differences of the exact projection); these tests
hold the HIP path to it at the fp64 / fp32 bars and repeat the known answers
through the C ABI.
"""

from dataclasses import replace

import numpy as np
import pytest

from oracle import projection as op
from purin_amd import workloads
from tests._gpu import canonical_from_workload, plan_for, rel_err, require_gpu, to_np
from tests._margins import Margins, check_counts, check_iterates

pytestmark = pytest.mark.gpu

TOL = {np.float64: 1e-10, np.float32: 1e-4}


def _per_sample(w, B, seed, spread=0.3):
    """Per-sample coefficients on the workload's sparsity, with a feasible point
    per sample: equality rhs K_b x0, inequality rhs K_b x0 + slack; singleton
    rows get per-sample coefficients of either sign."""
    canon = canonical_from_workload(w)
    support, mask, shared = canon.ell(np.float64)
    rng = np.random.default_rng(seed)
    values = shared[None] * (1 + spread * rng.uniform(-1, 1, (B,) + shared.shape))
    single = np.array([len(r) == 1 for r in canon.rows]) & (np.arange(len(canon.rows)) >= canon.me)
    values[:, single, 0] = rng.uniform(0.5, 2.0, (B, single.sum())) * rng.choice([-1, 1], (B, single.sum()))
    values = np.where(mask[None], values, 0)
    x0 = rng.uniform(-0.5, 0.5, (B, canon.n))
    Kx = np.sum(values * x0[:, support], axis=2)
    rhs = Kx.copy()
    rhs[:, canon.me:] += rng.uniform(0.2, 1.0, (B, len(canon.rows) - canon.me))
    return canon, values, rhs, mask


def _csr(values, mask):
    return np.ascontiguousarray(values[:, mask])


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("early_stop", [False, True])
@pytest.mark.parametrize("accelerated", [False, True])
def test_values_project_matches_oracle(dtype, early_stop, accelerated):
    require_gpu()
    B = 37
    w = workloads.small_random(31, n=40, me=6, mi=14, width=4, batch=B)
    canon, values, rhs, mask = _per_sample(w, B, 5)
    target = w.target.astype(dtype)
    iters = 600
    cfg = op.Config(accelerated=accelerated, max_iterations=iters, early_stop=early_stop,
                    tolerance=1e-6 if dtype == np.float64 else 1e-4)
    mg = Margins(
        lambda safety, tr: op.solve(canon, target, rhs.astype(dtype), replace(cfg, safety=safety),
                                    dtype=dtype, values=values.astype(dtype), trace=tr), dtype)
    want = mg.want
    plan = plan_for(canon, dtype=dtype, accelerated=accelerated)
    got = plan.project(target, rhs.astype(dtype), values=_csr(values, mask).astype(dtype),
                       tolerance=cfg.tolerance, max_iterations=iters, early_stop=early_stop,
                       check_every=7)
    bar = TOL[dtype]
    check_counts(to_np(got.iterations), mg)
    same = to_np(got.iterations) == want.iterations
    assert rel_err(to_np(got.y)[same], want.y[same]) <= bar
    assert rel_err(to_np(got.y), want.y) <= 10 * bar
    np.testing.assert_array_equal(to_np(got.status), want.status)
    mult = to_np(got.multipliers)
    want_mult = np.concatenate([want.multipliers_eq, want.multipliers_ineq], axis=1)
    assert rel_err(mult[same], want_mult[same]) <= TOL[dtype]
    assert rel_err(to_np(got.slacks)[same], want.slacks[same]) <= TOL[dtype]
    # the per-sample matrices differ: so do the per-sample iteration counts (the
    # accelerated fp64 case stays above the tolerance for the whole run)
    if early_stop and not accelerated:
        assert len(np.unique(want.iterations)) > 1


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("accelerated", [False, True])
def test_values_resident_matches_streaming_and_oracle(dtype, accelerated):
    """Fixed iterations with per-sample coefficients on the resident kernel:
    the iterate stays on chip and each tile streams its samples' scaled
    coefficients in the plan's stream order, with per-sample steps advanced in
    the kernel (kernels.py:209-227, 279-283).  Against the streaming passes on
    the whole batch and the oracle on two samples, for every slot count of the
    resident schedule (1, 2, 4 and 8 per thread)."""
    require_gpu()
    for k, (n, me, mi, width, B) in enumerate(((48, 8, 20, 4, 37), (700, 100, 300, 5, 40),
                                               (1500, 300, 700, 6, 24),
                                               (4096, 1024, 2048, 8, 12))):
        w = workloads.small_random(60 + k, n=n, me=me, mi=mi, width=width, batch=B,
                                   accelerated=accelerated)
        canon, values, rhs, mask = _per_sample(w, B, 70 + k)
        target = w.target.astype(dtype)
        rhs = rhs.astype(dtype)
        vals = _csr(values, mask).astype(dtype)
        plan = plan_for(canon, dtype=dtype, accelerated=accelerated)
        iters = 200
        kw = dict(values=vals, max_iterations=iters, early_stop=False, timing=True)
        print(f"values resident n={n} {np.dtype(dtype).name} accelerated={accelerated}",
              flush=True)
        res = plan.project(target, rhs, **kw)
        assert plan.last_timing()["resident"] == 1, n
        st = plan.project(target, rhs, streaming=True, **kw)
        assert plan.last_timing()["resident"] == 0, n
        bar = TOL[dtype]
        assert rel_err(to_np(res.y), to_np(st.y)) <= bar, n
        assert rel_err(to_np(res.multipliers), to_np(st.multipliers)) <= bar, n
        assert rel_err(to_np(res.slacks), to_np(st.slacks)) <= bar, n
        np.testing.assert_array_equal(to_np(res.status), to_np(st.status))
        sub = slice(0, 2)
        cfg = op.Config(accelerated=accelerated, max_iterations=iters, early_stop=False)
        want = op.solve(canon, target[sub], rhs[sub], cfg, dtype=dtype,
                        values=values[sub].astype(dtype))
        assert rel_err(to_np(res.y)[sub], want.y) <= bar, n
        want_mult = np.concatenate([want.multipliers_eq, want.multipliers_ineq], axis=1)
        assert rel_err(to_np(res.multipliers)[sub], want_mult) <= bar, n
        np.testing.assert_array_equal(to_np(res.status)[sub], want.status)


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("accelerated", [False, True])
def test_values_resident_early_stop(dtype, accelerated):
    """BoundProjection.solve's default loop (early stop, freezing,
    stationarity; kernels.py:238-290) with per-sample coefficients on the
    resident early-stop kernel.  fp64 counts equal the streaming passes' and
    the oracle's; fp32 counts follow the oracle under the rule of
    tests/_margins.py with the oracle's fp64 run on the same inputs among the
    perturbed runs, at tolerance 1e-2 (where the oracle's fp32 and fp64 runs
    stop every checked sample at the same iteration); same-count iterates at
    the parity bar, statuses equal."""
    require_gpu()
    tol = 1e-4 if dtype == np.float64 else 1e-2
    n_oracle = {48: 8, 700: 4, 1500: 3, 4096: 2}
    stopped = 0
    for k, (n, me, mi, width, B) in enumerate(((48, 8, 20, 4, 37), (700, 100, 300, 5, 40),
                                               (1500, 300, 700, 6, 24),
                                               (4096, 1024, 2048, 8, 12))):
        w = workloads.small_random(60 + k, n=n, me=me, mi=mi, width=width, batch=B,
                                   accelerated=accelerated)
        canon, values, rhs, mask = _per_sample(w, B, 70 + k)
        target = w.target.astype(dtype)
        rhs = rhs.astype(dtype)
        vals = _csr(values, mask).astype(dtype)
        plan = plan_for(canon, dtype=dtype, accelerated=accelerated)
        kw = dict(values=vals, max_iterations=2000, early_stop=True, tolerance=tol,
                  check_every=7, timing=True)
        print(f"values resident early stop n={n} {np.dtype(dtype).name} "
              f"accelerated={accelerated}", flush=True)
        res = plan.project(target, rhs, **kw)
        assert plan.last_timing()["resident"] == 1, n
        st = plan.project(target, rhs, streaming=True, **kw)
        assert plan.last_timing()["resident"] == 0, n
        it_r, it_s = to_np(res.iterations), to_np(st.iterations)
        bar = TOL[dtype]
        same = it_r == it_s
        if dtype == np.float64:
            np.testing.assert_array_equal(it_r, it_s)
        assert rel_err(to_np(res.y)[same], to_np(st.y)[same]) <= bar, n
        np.testing.assert_array_equal(to_np(res.status)[same], to_np(st.status)[same])
        stopped += int(np.sum(it_r < kw["max_iterations"]))
        sub = np.arange(n_oracle[n])
        cfg = op.Config(accelerated=accelerated, max_iterations=2000, early_stop=True,
                        tolerance=tol)
        v32 = values[sub].astype(dtype)
        alt = () if dtype == np.float64 else (
            lambda tr: op.solve(canon, target[sub].astype(np.float64),
                                rhs[sub].astype(np.float64), cfg, dtype=np.float64,
                                values=v32.astype(np.float64), trace=tr),)
        mg = Margins(lambda safety, tr: op.solve(canon, target[sub], rhs[sub],
                                                 replace(cfg, safety=safety), dtype=dtype,
                                                 values=v32, trace=tr), dtype, alternates=alt)
        print(f"  counts gpu {it_r[sub].tolist()} oracle {mg.want.iterations.tolist()}",
              flush=True)
        same_o = check_counts(it_r, mg, samples=sub)
        check_iterates(to_np(res.y), mg, same_o, bar, samples=sub)
        np.testing.assert_array_equal(to_np(res.status)[sub][same_o], mg.want.status[same_o])
    assert stopped > 0  # the stop test fired


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("mode", ["diagonal", "power"])
def test_values_steps_variants_match_oracle(dtype, mode):
    """Per-sample diagonal steps (kernels.py:76-88) and the per-sample
    power-iteration norm (norm_bound off, kernels.py:211-212)."""
    require_gpu()
    B = 29
    w = workloads.small_random(32, n=36, me=5, mi=12, width=3, batch=B)
    canon, values, rhs, mask = _per_sample(w, B, 6)
    target = w.target.astype(dtype)
    kw = dict(diagonal_preconditioning=True) if mode == "diagonal" else dict(norm_bound=False)
    cfg = op.Config(max_iterations=500, early_stop=True,
                    tolerance=1e-6 if dtype == np.float64 else 1e-4, **kw)
    mg = Margins(
        lambda safety, tr: op.solve(canon, target, rhs.astype(dtype), replace(cfg, safety=safety),
                                    dtype=dtype, values=values.astype(dtype), trace=tr), dtype)
    want = mg.want
    plan = plan_for(canon, dtype=dtype, **kw)
    got = plan.project(target, rhs.astype(dtype), values=_csr(values, mask).astype(dtype),
                       tolerance=cfg.tolerance, max_iterations=500, early_stop=True, check_every=5)
    check_counts(to_np(got.iterations), mg)
    same = to_np(got.iterations) == want.iterations
    assert rel_err(to_np(got.y)[same], want.y[same]) <= TOL[dtype]
    assert rel_err(to_np(got.y), want.y) <= 10 * TOL[dtype]
    np.testing.assert_array_equal(to_np(got.status), want.status)


def test_shared_values_match_the_shared_path():
    """values = the plan's own coefficients for every sample reproduce project()."""
    torch = require_gpu()
    B = 64
    w = workloads.config1(batch=B)
    canon = canonical_from_workload(w)
    _, mask, shared = canon.ell(np.float64)
    rhs = np.tile(w.rhs, (B, 1))
    plan = plan_for(canon, dtype=np.float64, accelerated=True)
    a = plan.project(w.target, rhs, max_iterations=300, early_stop=False, streaming=True)
    vals = np.broadcast_to(shared[mask], (B, int(mask.sum())))
    b = plan.project(w.target, rhs, values=vals, max_iterations=300, early_stop=False)
    assert rel_err(to_np(b.y), to_np(a.y)) <= 1e-12
    np.testing.assert_array_equal(to_np(b.status), to_np(a.status))
    assert torch.equal(b.iterations, a.iterations)


def test_values_vjp_matches_oracle_at_the_same_state():
    """g_target, g_rhs and g_values (the VJP of cp_step w.r.t. the scaled
    coefficients, chained through row scaling and the bound thresholds) at the
    GPU's converged state; converged GMRES at 1e-14."""
    require_gpu()
    B = 24
    dtype = np.float64
    w = workloads.small_random(33, n=20, me=3, mi=8, width=3, batch=B)
    canon, values, rhs, mask = _per_sample(w, B, 7)
    target = w.target
    cot = np.random.default_rng(9).normal(size=(B, canon.n))
    cfg = op.Config(max_iterations=20000, tolerance=1e-9, gmres_tolerance=1e-14,
                    gmres_max_iterations=300)
    plan = plan_for(canon, dtype=dtype)
    vcsr = _csr(values, mask)
    fwd = plan.project(target, rhs, values=vcsr, tolerance=cfg.tolerance,
                       max_iterations=cfg.max_iterations, save=True)
    status = to_np(fwd.status)
    assert np.sum(status == 0) >= B // 2
    pre = op.presolve(canon, rhs, cfg, dtype, values)
    dual = to_np(fwd.multipliers)[:, pre.rows] / pre.scale
    res, g_t, g_r, oadj, g_v = op.vjp(canon, target, rhs, cfg, cot, values=values,
                                      return_values=True, state=(to_np(fwd.y), dual))
    np.testing.assert_array_equal(status, res.status)
    adj = plan.adjoint(fwd.saved, None, None, cot, values=vcsr,
                       tolerance=cfg.gmres_tolerance, max_iterations=cfg.gmres_max_iterations)
    np.testing.assert_array_equal(to_np(adj.valid), oadj.valid)
    np.testing.assert_array_equal(to_np(adj.info), oadj.info)
    assert rel_err(to_np(adj.g_target), g_t) <= 1e-10
    assert rel_err(to_np(adj.g_rhs), g_r) <= 1e-10
    assert rel_err(to_np(adj.g_values), _csr(g_v, mask)) <= 1e-10
    assert np.abs(to_np(adj.g_values)).max() > 1e-3


@pytest.mark.parametrize("accelerated,diagonal", [(False, False), (True, False), (False, True)])
def test_values_parameter_coefficient_known_answer(accelerated, diagonal):
    """``a u + v == 1`` with a = 2 (reference tests/test_regression_chambolle_pock.py:116-137,
    tests/test_regression_cp_diagonal_steps.py:83-112): y and dy/da through the C ABI."""
    torch = require_gpu()
    from purin_amd.plan import Plan

    plan = Plan(2, 1, 0, np.array([0, 2]), np.array([0, 1]), np.array([1.0, 1.0]),
                dtype=torch.float64, accelerated=accelerated,
                diagonal_preconditioning=diagonal, device="cuda")
    a = 2.0
    x = np.array([[0.2, 0.3]])
    vals = np.array([[a, 1.0]])
    fwd = plan.project(x, np.array([[1.0]]), values=vals, save=True)
    f = (a * 0.2 + 0.3 - 1) / (a * a + 1)
    fp = (0.2 * (a * a + 1) - (a * 0.2 + 0.3 - 1) * 2 * a) / (a * a + 1) ** 2
    np.testing.assert_allclose(to_np(fwd.y)[0], [0.2 - a * f, 0.3 - f], atol=1e-8)
    jac = np.zeros(2)
    for k in range(2):
        cot = np.zeros((1, 2))
        cot[0, k] = 1.0
        jac[k] = to_np(plan.adjoint(fwd.saved, None, None, cot, values=vals).g_values)[0, 0]
    np.testing.assert_allclose(jac, [-(f + a * fp), -fp], atol=2e-7)


def test_values_bound_sign_zero_and_derivative():
    """``a u <= b`` (reference tests/test_regression_cp_bound_presolve.py:30-53)."""
    torch = require_gpu()
    from purin_amd.plan import Plan

    plan = Plan(1, 0, 1, np.array([0, 1]), np.array([0]), np.array([1.0]),
                dtype=torch.float64, device="cuda")
    x = np.array([[3.0], [-3.0], [3.0], [3.0]])
    theta = np.array([[2.0, 1.0], [-2.0, 1.0], [0.0, -1.0], [0.0, 1.0]])
    fwd = plan.project(x, theta[:, 1:], values=theta[:, :1], save=True)
    np.testing.assert_allclose(to_np(fwd.y), [[0.5], [-0.5], [3.0], [3.0]], atol=1e-10)
    assert to_np(fwd.eligible).tolist() == [True, True, False, True]
    adj = plan.adjoint(fwd.saved, None, None, np.ones((4, 1)), values=theta[:, :1])
    np.testing.assert_allclose(to_np(adj.g_values)[0, 0], -0.25, atol=1e-8)
    np.testing.assert_allclose(to_np(adj.g_rhs)[0, 0], 0.5, atol=1e-8)
    np.testing.assert_allclose(to_np(adj.g_target)[2], 0.0)
    np.testing.assert_allclose(to_np(adj.g_values)[2], 0.0)


def test_values_saved_state_and_option_errors():
    torch = require_gpu()
    from purin_amd import _lib
    from purin_amd.plan import Plan

    plan = Plan(2, 1, 0, np.array([0, 2]), np.array([0, 1]), np.array([1.0, 1.0]),
                dtype=torch.float64, device="cuda")
    x = np.array([[0.2, 0.3]])
    vals = np.array([[2.0, 1.0]])
    fwd = plan.project(x, np.array([[1.0]]), values=vals, save=True)
    with pytest.raises(_lib.PurinError, match="project_values"):
        plan.adjoint(fwd.saved, None, None, np.ones((1, 2)))
    plain = plan.project(x, np.array([[1.0]]), save=True)
    with pytest.raises(_lib.PurinError, match="not from"):
        plan.adjoint(plain.saved, None, None, np.ones((1, 2)), values=vals)
    with pytest.raises(_lib.PurinError, match="shared"):
        plan.project(x, np.array([[1.0]]), values=vals, shared_bounds=True)
    torch.cuda.synchronize()


@pytest.mark.parametrize("mode", ["scalar", "diagonal"])
def test_values_narrow_column_tiles(mode):
    """Per-sample coefficients on a network-flow problem (5000 nodes, 12000
    edges) whose wide column tile gathers more of d+ than an XCD's L2 holds:
    with B = 256 the fixed-iteration column pass takes a quarter wavefront per
    column, reading the per-sample coefficients and steps (scalar or diagonal)
    per lane.  The first 64 samples alone, a batch that runs the wide pass,
    give bit-identical results, and samples from both ends match the oracle."""
    require_gpu()
    B, k = 256, 64
    w = workloads.config3(batch=B, nodes=5000, edges=12000)
    canon = canonical_from_workload(w)
    support, mask, shared = canon.ell(np.float64)
    rng = np.random.default_rng(12)
    csr = shared[mask]
    vals = csr[None] * (1 + 0.3 * rng.uniform(-1, 1, (B, csr.size)))
    target = np.ascontiguousarray(w.target, np.float64)
    rhs = np.tile(w.rhs, (B, 1))
    kw = dict(diagonal_preconditioning=True) if mode == "diagonal" else {}
    plan = plan_for(canon, dtype=np.float64, **kw)
    opts = dict(max_iterations=120, early_stop=False)
    got = plan.project(target, rhs, values=vals, timing=True, **opts)
    t = plan.last_timing()
    assert t["resident"] == 0 and t["narrow_columns"] == 1
    wide = plan.project(target[:k], rhs[:k], values=np.ascontiguousarray(vals[:k]), timing=True,
                        **opts)
    assert plan.last_timing()["narrow_columns"] == 0
    np.testing.assert_array_equal(to_np(wide.y), to_np(got.y)[:k])
    np.testing.assert_array_equal(to_np(wide.multipliers), to_np(got.multipliers)[:k])
    pick = [0, B - 1]
    ell = np.zeros((len(pick),) + shared.shape)
    ell[:, mask] = vals[pick]
    cfg = op.Config(max_iterations=120, early_stop=False, **kw)
    want = op.solve(canon, target[pick], rhs[pick], cfg, dtype=np.float64, values=ell)
    assert rel_err(to_np(got.y)[pick], want.y) <= TOL[np.float64]
