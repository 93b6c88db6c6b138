"""GPU parity of the general diagonal QP (purin_cp_qp_solve / purin_cp_qp_adjoint)
with the oracle (oracle/diagonal_qp.py, the restatement of
src/purin/solvers/diagonal_qp.py:69-319), through the C ABI.

The oracle is pinned in tests/test_oracle_diagonal_qp.py (the reference's
known answer and differences of exact QP solutions).
"""

from dataclasses import replace

import numpy as np
import pytest

from oracle import diagonal_qp as dq
from oracle.cp import layout
from oracle.projection import Config
from tests._gpu import rel_err, require_gpu, to_np
from tests._margins import Margins, check_counts, check_iterates

pytestmark = pytest.mark.gpu

TOL = {np.float64: 1e-10, np.float32: 1e-4}


def _problem(seed, *, n=30, me=4, mi=10, width=4, B=33):
    """Random rows, per-sample q > 0, c, coefficients, feasible rhs and bounds
    (some infinite)."""
    rng = np.random.default_rng(seed)
    rows = [sorted(rng.choice(n, width, replace=False).tolist()) for _ in range(me + mi)]
    support, mask = layout(rows, n)
    values = np.where(mask[None], rng.normal(size=(B,) + mask.shape), 0)
    q = rng.uniform(0.5, 3.0, (B, n))
    c = rng.normal(size=(B, n)) * 2
    x0 = rng.uniform(-0.4, 0.4, (B, n))
    rhs = np.einsum("bmw,bmw->bm", values, x0[:, support])
    rhs[:, me:] += rng.uniform(0.1, 1.0, (B, mi))
    lower = np.where(rng.uniform(size=(B, n)) < 0.2, -np.inf, -0.8)
    upper = np.where(rng.uniform(size=(B, n)) < 0.2, np.inf, 0.8)
    return rows, me, mi, n, support, mask, dq.QPData(q, c, values, rhs, lower, upper)


def _plan(rows, me, mi, n, dtype, **kw):
    import torch
    from purin_amd.plan import Plan

    indptr = np.zeros(len(rows) + 1, np.int64)
    indptr[1:] = np.cumsum([len(r) for r in rows])
    indices = np.asarray([c for r in rows for c in r], np.int32)
    data = np.ones(indptr[-1])
    return Plan(n, me, mi, indptr, indices, data, dtype=torch.float64 if dtype == np.float64
                else torch.float32, bound_presolve=False, device="cuda", **kw)


def _cast(data, dtype):
    return dq.QPData(*(np.asarray(x, dtype) for x in data))


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("early_stop", [False, True])
@pytest.mark.parametrize("accelerated", [False, True])
def test_qp_solve_matches_oracle(dtype, early_stop, accelerated):
    require_gpu()
    rows, me, mi, n, support, mask, data = _problem(41)
    data = _cast(data, dtype)
    iters = 700
    # fp32: the gap's rounding error (sums of n objective terms of O(1)) is a
    # few percent of a 1e-4 tolerance, so stop decisions at 1e-4 are noise;
    # 1e-3 keeps them meaningful
    cfg = Config(accelerated=accelerated, max_iterations=iters, early_stop=early_stop,
                 tolerance=1e-6 if dtype == np.float64 else 1e-3)
    mg = Margins(lambda safety, tr: dq.solve(support, mask, me, data,
                                             replace(cfg, safety=safety), trace=tr), dtype)
    want = mg.want
    plan = _plan(rows, me, mi, n, dtype, accelerated=accelerated)
    got = plan.qp_solve(data.q, data.c, data.rhs, data.lower, data.upper,
                        values=data.values[:, mask], tolerance=cfg.tolerance,
                        max_iterations=iters, early_stop=early_stop, check_every=6)
    check_counts(to_np(got.iterations), mg)
    same = to_np(got.iterations) == want.iterations
    bar = TOL[dtype]
    assert rel_err(to_np(got.y)[same], want.y[same]) <= bar
    mult = to_np(got.multipliers)
    want_mult = np.concatenate([want.multipliers_eq, want.multipliers_ineq], axis=1)
    assert rel_err(mult[same], want_mult[same]) <= TOL[dtype]
    assert rel_err(to_np(got.slacks)[same], want.slacks[same]) <= TOL[dtype]
    np.testing.assert_array_equal(to_np(got.status), want.status)
    np.testing.assert_array_equal(to_np(got.converged), want.gradient_eligible)
    # the residual decides the status against the tolerance: fp64 agrees to 1e-6
    # relative; fp32 residuals near their rounding floor (~1e-5: stationarity
    # terms of O(10) at eps 6e-8 times the row length) agree to 5 % of the tolerance
    gr, wr = to_np(got.residual)[same], want.residual_inf_norm[same]
    if dtype == np.float64:
        assert rel_err(gr, wr) <= 1e-6
    else:
        np.testing.assert_allclose(gr, wr, rtol=0, atol=0.05 * cfg.tolerance)
    if early_stop and not accelerated:
        assert len(np.unique(want.iterations)) > 1


# sizes (n, me, mi, width, B) covering every slot count of the resident
# schedule (1, 2, 4 and 8 row and column slots per thread)
RESIDENT_QP_SIZES = ((30, 4, 10, 4, 33), (700, 100, 300, 5, 40), (1500, 300, 700, 6, 24),
                     (4096, 1024, 2048, 8, 12))


def _shared_qp(n, me, mi, width, B, dtype, accelerated):
    """A QP whose coefficients are the plan's own (one set for the batch):
    per-sample q, c, rhs, bounds (some infinite) and a warm start y0."""
    import torch
    from purin_amd.plan import Plan

    rng = np.random.default_rng(n + 7)
    rows = [sorted(rng.choice(n, width, replace=False).tolist()) for _ in range(me + mi)]
    support, mask = layout(rows, n)
    coef = np.where(mask, rng.normal(size=mask.shape), 0)
    values = np.broadcast_to(coef, (B,) + mask.shape)
    q = rng.uniform(0.5, 3.0, (B, n))
    c = rng.normal(size=(B, n)) * 2
    x0 = rng.uniform(-0.4, 0.4, (B, n))
    rhs = np.einsum("bmw,bmw->bm", values, x0[:, support])
    rhs[:, me:] += rng.uniform(0.1, 1.0, (B, mi))
    lower = np.where(rng.uniform(size=(B, n)) < 0.2, -np.inf, -0.8)
    upper = np.where(rng.uniform(size=(B, n)) < 0.2, np.inf, 0.8)
    y0 = rng.uniform(-0.5, 0.5, (B, n)).astype(dtype)
    data = _cast(dq.QPData(q, c, values, rhs, lower, upper), dtype)
    indptr = np.zeros(len(rows) + 1, np.int64)
    indptr[1:] = np.cumsum([len(r) for r in rows])
    indices = np.asarray([j for r in rows for j in r], np.int32)
    plan = Plan(n, me, mi, indptr, indices, coef[mask], bound_presolve=False,
                dtype=torch.float64 if dtype == np.float64 else torch.float32,
                accelerated=accelerated, device="cuda")
    return support, mask, data, y0, plan


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("accelerated", [False, True])
def test_qp_resident_matches_streaming_and_oracle(dtype, accelerated):
    """Fixed iterations of the diagonal QP on the resident kernel (per-sample q
    and c in registers, per-sample steps advanced in the kernel as the
    streaming passes' schedule does, kernels.py:279-283 with gamma = min q):
    against the streaming passes on the whole batch and the oracle on two
    samples, for every slot count of the resident schedule, with a warm
    start, random boxes, one shared box, and per-sample coefficients."""
    require_gpu()
    for n, me, mi, width, B in RESIDENT_QP_SIZES:
        support, mask, data, y0, plan = _shared_qp(n, me, mi, width, B, dtype, accelerated)
        iters = 300
        kw = dict(max_iterations=iters, early_stop=False, y0=y0, timing=True)
        print(f"QP resident n={n} {np.dtype(dtype).name} accelerated={accelerated}", flush=True)
        res = plan.qp_solve(data.q, data.c, data.rhs, data.lower, data.upper, **kw)
        assert plan.last_timing()["resident"] == 1, n
        st = plan.qp_solve(data.q, data.c, data.rhs, data.lower, data.upper, streaming=True, **kw)
        assert plan.last_timing()["resident"] == 0, n
        bar = TOL[dtype]
        assert rel_err(to_np(res.y), to_np(st.y)) <= bar, n
        assert rel_err(to_np(res.multipliers), to_np(st.multipliers)) <= bar, n
        assert rel_err(to_np(res.slacks), to_np(st.slacks)) <= bar, n
        np.testing.assert_array_equal(to_np(res.status), to_np(st.status))
        np.testing.assert_array_equal(to_np(res.iterations), iters)
        sub = slice(0, 2)
        cfg = Config(accelerated=accelerated, max_iterations=iters, early_stop=False)
        want = dq.solve(support, mask, me, dq.QPData(*(x[sub] for x in data)), cfg,
                        y0=y0[sub])
        assert rel_err(to_np(res.y)[sub], want.y) <= bar, n
        want_mult = np.concatenate([want.multipliers_eq, want.multipliers_ineq], axis=1)
        assert rel_err(to_np(res.multipliers)[sub], want_mult) <= bar, n
        np.testing.assert_array_equal(to_np(res.status)[sub], want.status)
        y, lo, hi = to_np(res.y)[sub], data.lower[sub], data.upper[sub]
        np.testing.assert_array_equal(y == lo, want.y == lo)
        np.testing.assert_array_equal(y == hi, want.y == hi)
        # one box for every sample and column: the kernel holds it in registers
        box = np.full((B, n), 0.8, dtype)
        rb = plan.qp_solve(data.q, data.c, data.rhs, -box, box, **kw)
        assert plan.last_timing()["resident"] == 1, n
        sb = plan.qp_solve(data.q, data.c, data.rhs, -box, box, streaming=True, **kw)
        assert rel_err(to_np(rb.y), to_np(sb.y)) <= bar, n
        assert rel_err(to_np(rb.multipliers), to_np(sb.multipliers)) <= bar, n
        np.testing.assert_array_equal(to_np(rb.y) == 0.8, to_np(sb.y) == 0.8)
        # per-sample coefficients (the front end's call): each tile streams its
        # samples' coefficients
        scale = np.random.default_rng(n).uniform(0.8, 1.2, data.values.shape)
        pv = (data.values * scale).astype(dtype)
        rv = plan.qp_solve(data.q, data.c, data.rhs, data.lower, data.upper, values=pv[:, mask],
                           **kw)
        assert plan.last_timing()["resident"] == 1, n
        sv = plan.qp_solve(data.q, data.c, data.rhs, data.lower, data.upper, values=pv[:, mask],
                           streaming=True, **kw)
        assert rel_err(to_np(rv.y), to_np(sv.y)) <= bar, n
        assert rel_err(to_np(rv.multipliers), to_np(sv.multipliers)) <= bar, n
        wantv = dq.solve(support, mask, me, dq.QPData(*(x[sub] for x in data._replace(values=pv))),
                         cfg, y0=y0[sub])
        assert rel_err(to_np(rv.y)[sub], wantv.y) <= bar, n


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("accelerated", [False, True])
def test_qp_resident_early_stop(dtype, accelerated):
    """PreparedDiagonalQP.solve's default loop (early stop, freezing,
    stationarity; kernels.py:238-290 with general q, c) on the resident
    kernel: each sample stops on its own.  fp64 iteration counts equal the
    streaming passes' and the oracle's; fp32 counts follow the oracle under
    the rule of tests/_margins.py, with the oracle's fp64 run on the same
    inputs among the perturbed runs; same-count iterates and multipliers at
    the parity bar; statuses equal."""
    require_gpu()
    # fp32 at 1e-2: there the oracle's fp32 and fp64 runs stop every sample at
    # the same iteration, with margins 1e-4 to 1e-3 apart at the stop.  At 1e-3
    # the accelerated n = 4096 samples' margins fall by ~10 % per iteration
    # through 1 and sit ~1.5 % apart between the oracle's fp32 and fp64 runs
    # and ~6 % between the oracle and this kernel (its K ybar from K y, its sums
    # in scheduled order), so rounding, not the recurrence, picks the
    # iteration there.
    tol = 1e-6 if dtype == np.float64 else 1e-2
    n_oracle = {30: 8, 700: 4, 1500: 3, 4096: 2}
    stopped = 0
    for n, me, mi, width, B in RESIDENT_QP_SIZES:
        support, mask, data, y0, plan = _shared_qp(n, me, mi, width, B, dtype, accelerated)
        kw = dict(max_iterations=2000, early_stop=True, tolerance=tol, y0=y0, check_every=7,
                  timing=True)
        print(f"QP resident early stop n={n} {np.dtype(dtype).name} accelerated={accelerated}",
              flush=True)
        res = plan.qp_solve(data.q, data.c, data.rhs, data.lower, data.upper, **kw)
        assert plan.last_timing()["resident"] == 1, n
        st = plan.qp_solve(data.q, data.c, data.rhs, data.lower, data.upper, streaming=True, **kw)
        assert plan.last_timing()["resident"] == 0, n
        it_r, it_s = to_np(res.iterations), to_np(st.iterations)
        bar = TOL[dtype]
        same = it_r == it_s
        if dtype == np.float64:
            np.testing.assert_array_equal(it_r, it_s)
        assert rel_err(to_np(res.y)[same], to_np(st.y)[same]) <= bar, n
        assert rel_err(to_np(res.multipliers)[same], to_np(st.multipliers)[same]) <= bar, n
        np.testing.assert_array_equal(to_np(res.status)[same], to_np(st.status)[same])
        stopped += int(np.sum(it_r < kw["max_iterations"]))
        sub = np.arange(n_oracle[n])
        cfg = Config(accelerated=accelerated, max_iterations=kw["max_iterations"],
                     early_stop=True, tolerance=tol)
        part = dq.QPData(*(x[sub] for x in data))
        # fp32: the oracle in fp64 on the same (fp32) inputs measures the
        # rounding noise of the stop margin (the gap's objective sums)
        part64 = dq.QPData(*(np.asarray(x, np.float64) for x in part))
        alt = () if dtype == np.float64 else (
            lambda tr: dq.solve(support, mask, me, part64, cfg,
                                y0=y0[sub].astype(np.float64), trace=tr),)
        mg = Margins(lambda safety, tr: dq.solve(support, mask, me, part,
                                                 replace(cfg, safety=safety), y0=y0[sub],
                                                 trace=tr), dtype, alternates=alt)
        print(f"  counts gpu {it_r[sub].tolist()} oracle {mg.want.iterations.tolist()}",
              flush=True)
        same_o = check_counts(it_r, mg, samples=sub)
        check_iterates(to_np(res.y), mg, same_o, bar, samples=sub)
        np.testing.assert_array_equal(to_np(res.status)[sub][same_o], mg.want.status[same_o])
    assert stopped > 0  # the stop test fired


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("mode", ["diagonal", "power"])
def test_qp_step_variants_match_oracle(dtype, mode):
    """Per-variable diagonal steps (q does not enter them, kernels.py:76-88) and
    the power-iteration norm (norm_bound off)."""
    require_gpu()
    rows, me, mi, n, support, mask, data = _problem(42, B=21)
    data = _cast(data, dtype)
    kw = dict(diagonal_preconditioning=True) if mode == "diagonal" else dict(norm_bound=False)
    cfg = Config(max_iterations=500, early_stop=False,
                 tolerance=1e-6 if dtype == np.float64 else 1e-4, **kw)
    want = dq.solve(support, mask, me, data, cfg)
    plan = _plan(rows, me, mi, n, dtype, **kw)
    got = plan.qp_solve(data.q, data.c, data.rhs, data.lower, data.upper,
                        values=data.values[:, mask], tolerance=cfg.tolerance,
                        max_iterations=500, early_stop=False)
    assert rel_err(to_np(got.y), want.y) <= TOL[dtype]
    np.testing.assert_array_equal(to_np(got.status), want.status)


@pytest.mark.parametrize("early_stop", [False, True])
def test_qp_shared_values_and_warm_start(early_stop):
    """values = None uses the plan's coefficients for every sample; a warm start
    (y0, dual0) enters the iteration like the oracle's (diagonal_qp.py:240-273).
    The shared streaming path reads one copy of the scaled entries, the same
    bits as every sample's copy when the values are passed per sample, so the
    two agree exactly.  (By default both run on the resident kernel, which
    sums in its own scheduled order: held to the oracle at the parity bar.)"""
    require_gpu()
    rows, me, mi, n, support, mask, data = _problem(43, B=17)
    shared = data.values[0]
    data = data._replace(values=np.broadcast_to(shared, data.values.shape).copy())
    x0 = np.random.default_rng(1).uniform(-0.4, 0.4, (17, n))
    data = data._replace(rhs=np.einsum("mw,bmw->bm", shared, x0[:, support]) + np.concatenate(
        (np.zeros((17, me)), np.full((17, mi), 0.3)), axis=1))
    from purin_amd.plan import Plan
    import torch

    indptr = np.zeros(len(rows) + 1, np.int64)
    indptr[1:] = np.cumsum([len(r) for r in rows])
    indices = np.asarray([c for r in rows for c in r], np.int32)
    plan = Plan(n, me, mi, indptr, indices, shared[mask], dtype=torch.float64,
                bound_presolve=False, device="cuda")
    iters = 2000 if early_stop else 300
    cfg = Config(max_iterations=iters, early_stop=early_stop)
    y0 = np.random.default_rng(2).uniform(-0.5, 0.5, (17, n))
    d0 = np.random.default_rng(3).normal(size=(17, me + mi))
    d0[:, me:] = np.abs(d0[:, me:])
    want = dq.solve(support, mask, me, data, cfg, y0=y0, dual0=d0)
    got = plan.qp_solve(data.q, data.c, data.rhs, data.lower, data.upper, y0=y0, dual0=d0,
                        max_iterations=iters, early_stop=early_stop)
    assert rel_err(to_np(got.y), want.y) <= 1e-10
    got_s = plan.qp_solve(data.q, data.c, data.rhs, data.lower, data.upper, y0=y0, dual0=d0,
                          max_iterations=iters, early_stop=early_stop, streaming=True)
    assert rel_err(to_np(got_s.y), want.y) <= 1e-10
    got2 = plan.qp_solve(data.q, data.c, data.rhs, data.lower, data.upper, y0=y0, dual0=d0,
                         values=data.values[:, mask], max_iterations=iters,
                         early_stop=early_stop, streaming=True)
    np.testing.assert_array_equal(to_np(got2.y), to_np(got_s.y))
    np.testing.assert_array_equal(to_np(got2.iterations), to_np(got_s.iterations))


@pytest.mark.parametrize("mode", ["scalar", "diagonal"])
def test_qp_vjp_matches_oracle_at_the_same_state(mode):
    """All six gradients and the dual cotangent's path at the GPU's converged
    state; converged GMRES at 1e-14."""
    require_gpu()
    rows, me, mi, n, support, mask, data = _problem(44, n=16, me=2, mi=5, width=3, B=20)
    kw = dict(diagonal_preconditioning=True) if mode == "diagonal" else {}
    cfg = Config(max_iterations=30000, tolerance=1e-9, gmres_tolerance=1e-14,
                 gmres_max_iterations=300, **kw)
    plan = _plan(rows, me, mi, n, np.float64, **kw)
    vals = data.values[:, mask]
    fwd = plan.qp_solve(data.q, data.c, data.rhs, data.lower, data.upper, values=vals,
                        tolerance=cfg.tolerance, max_iterations=cfg.max_iterations, save=True)
    status = to_np(fwd.status)
    assert np.sum(status == 0) >= 10
    rng = np.random.default_rng(5)
    cot = rng.normal(size=(20, n))
    cot_dual = rng.normal(size=(20, me + mi))
    scale = dq._scale(data._replace(values=np.where(mask[None], data.values, 0)), mask, cfg)
    dual = to_np(fwd.multipliers) / scale
    res, g, oadj = dq.vjp(support, mask, me, data, cfg, cot, cot_dual,
                          state=(to_np(fwd.y), dual))
    np.testing.assert_array_equal(status, res.status)
    adj = plan.qp_adjoint(fwd.saved, data.q, data.c, cot, values=vals, cot_dual=cot_dual,
                          tolerance=cfg.gmres_tolerance, max_iterations=cfg.gmres_max_iterations)
    np.testing.assert_array_equal(to_np(adj.valid), oadj.valid)
    np.testing.assert_array_equal(to_np(adj.info), oadj.info)
    for name, want in (("g_q", g.q), ("g_c", g.c), ("g_rhs", g.rhs), ("g_lower", g.lower),
                       ("g_upper", g.upper), ("g_values", g.values[:, mask])):
        assert rel_err(to_np(getattr(adj, name)), want) <= 1e-10, name
    assert np.abs(to_np(adj.g_q)).max() > 1e-3


@pytest.mark.parametrize("mode", ["scalar", "diagonal"])
def test_qp_adjoint_shared_values_equal_per_sample(mode):
    """The QP's VJP with the plan's own coefficients (values = None: one shared
    copy of the scaled entries) equals, bit for bit, the VJP with those
    coefficients passed per sample (both forwards on the streaming passes,
    which read the shared copy in the per-sample order)."""
    require_gpu()
    rows, me, mi, n, support, mask, data = _problem(45, n=16, me=2, mi=5, width=3, B=20)
    shared = data.values[0]
    data = data._replace(values=np.broadcast_to(shared, data.values.shape).copy())
    x0 = np.random.default_rng(6).uniform(-0.4, 0.4, (20, n))
    data = data._replace(rhs=np.einsum("mw,bmw->bm", shared, x0[:, support]) + np.concatenate(
        (np.zeros((20, me)), np.full((20, mi), 0.3)), axis=1))
    kw = dict(diagonal_preconditioning=True) if mode == "diagonal" else {}
    from purin_amd.plan import Plan
    import torch

    indptr = np.zeros(len(rows) + 1, np.int64)
    indptr[1:] = np.cumsum([len(r) for r in rows])
    indices = np.asarray([c for r in rows for c in r], np.int32)
    plan = Plan(n, me, mi, indptr, indices, shared[mask], dtype=torch.float64,
                bound_presolve=False, device="cuda", **kw)
    rng = np.random.default_rng(7)
    cot = rng.normal(size=(20, n))
    cot_dual = rng.normal(size=(20, me + mi))
    outs = []
    for vals in (None, data.values[:, mask]):
        fwd = plan.qp_solve(data.q, data.c, data.rhs, data.lower, data.upper, values=vals,
                            tolerance=1e-9, max_iterations=20000, save=True, streaming=True)
        adj = plan.qp_adjoint(fwd.saved, data.q, data.c, cot, values=vals, cot_dual=cot_dual,
                              tolerance=1e-12, max_iterations=200)
        outs.append((fwd, adj))
    (f0, a0), (f1, a1) = outs
    np.testing.assert_array_equal(to_np(f0.y), to_np(f1.y))
    for name in ("g_q", "g_c", "g_rhs", "g_lower", "g_upper"):
        np.testing.assert_array_equal(to_np(getattr(a0, name)), to_np(getattr(a1, name)), name)
    np.testing.assert_array_equal(to_np(a0.info), to_np(a1.info))


@pytest.mark.parametrize("accelerated", [False, True])
@pytest.mark.parametrize("scaling", [False, True])
def test_qp_known_answer(accelerated, scaling):
    """Reference tests/test_diagonal_qp.py:13-48: q = [2, 4], c = [-2, -4],
    u + v = 1 gives [1/3, 2/3]; dy/dc = -Q^-1 + Q^-1 a (a'Q^-1 a)^-1 a'Q^-1."""
    torch = require_gpu()
    from purin_amd.plan import Plan

    plan = Plan(2, 1, 0, np.array([0, 2]), np.array([0, 1]), np.array([1.0, 1.0]),
                dtype=torch.float64, accelerated=accelerated, row_scaling=scaling,
                bound_presolve=False, device="cuda")
    q, c = np.array([[2.0, 4.0]]), np.array([[-2.0, -4.0]])
    inf = np.full((1, 2), np.inf)
    fwd = plan.qp_solve(q, c, np.array([[1.0]]), -inf, inf, max_iterations=3000, save=True)
    np.testing.assert_allclose(to_np(fwd.y), [[1 / 3, 2 / 3]], atol=1e-8)
    assert to_np(fwd.residual)[0] < 1e-8
    jac = np.zeros((2, 2))
    for k in range(2):
        cot = np.zeros((1, 2))
        cot[0, k] = 1.0
        jac[k] = to_np(plan.qp_adjoint(fwd.saved, q, c, cot).g_c)[0]
    expected = -np.diag([0.5, 0.25]) + np.outer([0.5, 0.25], [0.5, 0.25]) / 0.75
    np.testing.assert_allclose(jac, expected, atol=1e-7)
    warm = plan.qp_solve(q, c, np.array([[1.0]]), -inf, inf, y0=fwd.y, dual0=fwd.multipliers,
                         max_iterations=3000)
    np.testing.assert_allclose(to_np(warm.y), to_np(fwd.y), atol=1e-8)


def test_qp_argument_errors():
    torch = require_gpu()
    from purin_amd import _lib
    from purin_amd.plan import Plan

    q, c = np.array([[2.0, 4.0]]), np.array([[-2.0, -4.0]])
    inf = np.full((1, 2), np.inf)
    presolving = Plan(2, 1, 0, np.array([0, 2]), np.array([0, 1]), np.array([1.0, 1.0]),
                      dtype=torch.float64, device="cuda")
    with pytest.raises(_lib.PurinError, match="bound_presolve"):
        presolving.qp_solve(q, c, np.array([[1.0]]), -inf, inf)
    plan = Plan(2, 1, 0, np.array([0, 2]), np.array([0, 1]), np.array([1.0, 1.0]),
                dtype=torch.float64, bound_presolve=False, device="cuda")
    fwd = plan.qp_solve(q, c, np.array([[1.0]]), -inf, inf, save=True)
    with pytest.raises(_lib.PurinError, match="qp_adjoint"):
        plan.adjoint(fwd.saved, None, None, np.ones((1, 2)))
    proj = plan.project(np.zeros((1, 2)), np.array([[1.0]]), save=True)
    with pytest.raises(_lib.PurinError, match="not from purin_cp_qp_solve"):
        plan.qp_adjoint(proj.saved, q, c, np.ones((1, 2)))
    torch.cuda.synchronize()
