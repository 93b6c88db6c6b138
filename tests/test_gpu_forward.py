"""GPU parity of the forward path: HIP kernels (through the C ABI) vs the CPU oracle.

Bars (from the task): relative error <= 1e-10 in fp64 and <= 1e-4 in fp32 on
projected points and multipliers; identical iteration counts, status codes and
active-set masks.  Relative error is ``max|a-b| / max|b|``.
"""

from dataclasses import replace

import numpy as np
import pytest

from oracle import cp as ocp
from oracle import projection as op
from purin_amd import workloads
from tests import _cases
from tests._gpu import canonical_from_workload, plan_for, rel_err, require_gpu, to_np
from tests._margins import Margins, check_counts, check_iterates

pytestmark = pytest.mark.gpu

TOL = {np.float64: 1e-10, np.float32: 1e-4}


def _kept(canon, rhs, dtype, cfg=op.Config()):
    return op.presolve(canon, rhs, cfg, dtype)


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("transpose", [False, True])
@pytest.mark.parametrize("scaled", [True, False])
def test_spmm_matches_oracle(dtype, transpose, scaled):
    torch = require_gpu()
    w = workloads.config1(batch=37)
    canon = canonical_from_workload(w)
    plan = plan_for(canon, dtype=dtype)
    rhs = np.tile(w.rhs, (37, 1)).astype(dtype)
    pre = _kept(canon, rhs, dtype)
    ksup, kmask = pre.support[pre.rows], pre.mask[pre.rows]
    values = pre.kept_values[0] if scaled else pre.values[pre.rows]
    mv, tmv = ocp.operators(values, ksup, kmask, canon.n)
    rng = np.random.default_rng(0)
    x = rng.normal(size=(37, len(pre.rows) if transpose else canon.n)).astype(dtype)
    want = tmv(x) if transpose else mv(x)
    got = to_np(plan.spmm(torch.as_tensor(x), transpose=transpose, scaled=scaled))
    assert rel_err(got, want) <= (1e-14 if dtype == np.float64 else 1e-6)
    np.testing.assert_allclose(plan.row_scale, pre.scale[0], rtol=1e-15 if dtype == np.float64 else 1e-7)


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("accelerated", [False, True])
@pytest.mark.parametrize("early_stop", [False, True])
def test_solve_matches_oracle(dtype, accelerated, early_stop):
    torch = require_gpu()
    B = 50
    w = workloads.small_random(11, n=48, me=8, mi=20, width=4, batch=B)
    canon = canonical_from_workload(w)
    rhs = np.tile(w.rhs, (B, 1)).astype(dtype)
    target = w.target.astype(dtype)
    pre = _kept(canon, rhs, dtype)
    ksup, kmask = pre.support[pre.rows], pre.mask[pre.rows]
    iters = 400
    tol = 1e-6 if dtype == np.float64 else 1e-4
    mg = Margins(lambda safety, tr: ocp.sparse_cp(
        np.ones_like(target), -target, pre.kept_values[0], pre.kept_rhs, ksup, kmask, canon.me,
        pre.lower, pre.upper, accelerated=accelerated, safety=safety, max_iterations=iters,
        tolerance=tol, y0=target, freeze_converged=True, check_stationarity=True,
        norm_bound=True, early_stop=early_stop, trace=tr), dtype)
    want = mg.want
    plan = plan_for(canon, dtype=dtype, accelerated=accelerated)
    got = plan.solve(pre.kept_rhs, target, pre.lower, pre.upper, tolerance=tol,
                     max_iterations=iters, early_stop=early_stop, check_every=7)
    bar = TOL[dtype]
    # counts: identical in fp64; in fp32 a sample may stop elsewhere only where
    # the oracle's own stop is borderline (tests/_margins.py)
    same = check_counts(to_np(got.iterations), mg)
    check_iterates(to_np(got.y), mg, same, bar)
    assert rel_err(to_np(got.dual)[same], want.dual[same]) <= bar
    np.testing.assert_array_equal(to_np(got.converged)[same], want.converged[same])
    # diagnostics of a nearly converged iterate sit near the rounding floor in fp32
    dtol = dict(rtol=1e-6, atol=1e-12) if dtype == np.float64 else dict(rtol=1e-2, atol=2e-5)
    np.testing.assert_allclose(to_np(got.residual)[same], want.residual[same], **dtol)
    np.testing.assert_allclose(to_np(got.gap)[same], want.gap[same], **dtol)
    if early_stop and not accelerated:
        assert np.any(want.iterations < iters), "the stop test should fire for some samples"
    # active sets on same-count samples: bound activity and positive inequality duals
    y, d = to_np(got.y)[same], to_np(got.dual)[same]
    lo, hi = pre.lower[same], pre.upper[same]
    np.testing.assert_array_equal(y == lo, want.y[same] == lo)
    np.testing.assert_array_equal(y == hi, want.y[same] == hi)
    np.testing.assert_array_equal(d[:, canon.me:] > 0, want.dual[same][:, canon.me:] > 0)


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("accelerated", [False, True])
def test_project_config1_fixed_iterations(dtype, accelerated):
    """Config 1 (n=64, 16+32 rows, B=32, 1000 fixed iterations) through purin_cp_project."""
    torch = require_gpu()
    w = workloads.config1()
    canon = canonical_from_workload(w)
    B = w.batch
    rhs = np.tile(w.rhs, (B, 1)).astype(dtype)
    target = w.target.astype(dtype)
    cfg = op.Config(accelerated=accelerated, max_iterations=1000, early_stop=False)
    want = op.solve(canon, target, rhs, cfg, dtype=dtype)
    plan = plan_for(canon, dtype=dtype, accelerated=accelerated)
    got = plan.project(target, rhs, max_iterations=1000, early_stop=False)
    bar = TOL[dtype]
    assert rel_err(to_np(got.y), want.y) <= bar
    mult = np.concatenate((want.multipliers_eq, want.multipliers_ineq), axis=1)
    assert rel_err(to_np(got.multipliers), mult) <= bar
    assert rel_err(to_np(got.slacks), want.slacks) <= bar
    np.testing.assert_array_equal(to_np(got.status), want.status)
    np.testing.assert_array_equal(to_np(got.iterations), want.iterations)
    np.testing.assert_array_equal(to_np(got.finite), want.finite)
    np.testing.assert_array_equal(to_np(got.eligible), want.gradient_eligible)
    np.testing.assert_allclose(to_np(got.residual), want.residual_inf_norm,
                               **(dict(rtol=1e-5, atol=1e-13) if dtype == np.float64
                                  else dict(rtol=1e-2, atol=2e-5)))
    np.testing.assert_array_equal(to_np(got.multipliers)[:, canon.me:] > 0, mult[:, canon.me:] > 0)


@pytest.mark.parametrize("shared", [False, True])
def test_project_early_stop_counts_and_statuses(shared):
    torch = require_gpu()
    B = 77
    w = workloads.small_random(5, n=40, me=6, mi=14, width=3, batch=B)
    canon = canonical_from_workload(w)
    rhs = np.tile(w.rhs, (B, 1))
    cfg = op.Config(max_iterations=3000, tolerance=1e-8)
    want = op.solve(canon, w.target, rhs, cfg)
    plan = plan_for(canon, dtype=np.float64)
    got = plan.project(w.target, rhs, max_iterations=3000, tolerance=1e-8, shared_bounds=shared,
                       check_every=16)
    np.testing.assert_array_equal(to_np(got.iterations), want.iterations)
    np.testing.assert_array_equal(to_np(got.status), want.status)
    assert np.any(want.status == op.CONVERGED)
    assert rel_err(to_np(got.y), want.y) <= 1e-10


def _kn(canon, target, rhs, **cfgkw):
    torch = require_gpu()
    cfg = op.Config(**cfgkw)
    plan = plan_for(canon, dtype=np.float64, accelerated=cfg.accelerated)
    got = plan.project(np.asarray(target, np.float64), np.asarray(rhs, np.float64),
                       max_iterations=cfg.max_iterations, tolerance=cfg.tolerance)
    return got, op.solve(canon, target, rhs, cfg)


@pytest.mark.parametrize("accelerated", [False, True])
def test_known_answer_affine_projection(accelerated):
    """Reference tests/test_regression_chambolle_pock.py:25-38."""
    got, want = _kn(_cases.sum_equals_b_u_nonneg(), [[2.0, 0.0], [-2.0, 0.0]],
                    [[1.0, 0.0], [1.0, 0.0]], accelerated=accelerated)
    np.testing.assert_allclose(to_np(got.y), [[1.5, -0.5], [0.0, 1.0]], atol=1e-8)
    assert np.all(to_np(got.status) == 0)
    assert np.max(to_np(got.residual)) <= 1e-9
    np.testing.assert_array_equal(to_np(got.iterations), want.iterations)


def test_known_answer_tied_bounds_multipliers_slacks():
    """Reference tests/test_regression_cp_bound_presolve.py:13-24 (no kept rows at all)."""
    canon, rhs = _cases.tied_scaled_bounds()
    got, want = _kn(canon, [[-3.0, 4.0]], rhs[None])
    np.testing.assert_allclose(to_np(got.y), [[0.0, 1.0]], atol=1e-10)
    np.testing.assert_allclose(to_np(got.multipliers), [[1.5, 0.75, 0.0, 3.0]], atol=1e-9)
    np.testing.assert_allclose(to_np(got.slacks), [[0.0, 0.0, 2.0, 0.0]], atol=1e-10)
    assert to_np(got.status)[0] == 0


def test_known_answer_status_codes():
    """Reference tests/test_regression_chambolle_pock.py:68-85, 140-164."""
    canon = _cases.sum_equals_b_u_nonneg()
    got, _ = _kn(canon, [[-2.0, 0.0]], [[1.0, 0.0]], max_iterations=1)
    assert to_np(got.status)[0] == 1 and not to_np(got.eligible)[0]
    got, _ = _kn(canon, [[np.nan, 0.0]], [[1.0, 0.0]], max_iterations=1)
    assert to_np(got.status)[0] == 3
    infeasible = _cases.canonical_from_dense(np.zeros((0, 1)), [[1.0], [-1.0]], 1)
    got, _ = _kn(infeasible, [[0.0]], [[0.0, -1.0]], max_iterations=100)
    assert to_np(got.status)[0] == 1 and not to_np(got.eligible)[0]
    scaled = _cases.canonical_from_dense([[1000.0, 1000.0]], [[-1.0, 0.0]], 2)
    got, _ = _kn(scaled, [[2.0, 0.0]], [[1000.0, 0.0]])
    assert to_np(got.eligible)[0]
    assert abs(float(to_np(got.y).sum()) * 1000 - 1000) <= 1e-9


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_crossed_bounds_keep_running_under_early_stop(dtype):
    """Samples whose bound rows cross (y0 <= 0 and y0 >= 1: lower > upper) are
    infeasible; the reference's stop test sees their bound violation
    (kernels.py:158-175) and never accepts them, so they run to
    max_iterations with status 1, beside feasible samples of the same batch
    (y0 in [-1, 1]) that stop on their own.  The resident early-stop kernel
    (which drops the violation term on lanes whose bounds cannot be violated)
    and the streaming passes against the oracle."""
    require_gpu()
    canon = _cases.canonical_from_dense([[1.0, 1.0]], [[1.0, 0.0], [-1.0, 0.0]], 2)
    B = 6
    target = np.array([[0.3, 0.2], [0.5, -0.1], [2.0, 1.0], [-1.0, 0.4], [0.9, 0.9],
                       [-2.0, 0.5]], dtype)
    rhs = np.array([[0.5, 0.0, -1.0] if s % 2 == 0 else [0.5, 1.0, 1.0] for s in range(B)],
                   dtype)
    crossed = np.arange(B) % 2 == 0
    cfg = op.Config(max_iterations=500, tolerance=1e-6)
    want = op.solve(canon, target, rhs, cfg, dtype=dtype)
    assert np.all(want.iterations[crossed] == 500)
    assert np.all(want.iterations[~crossed] < 500)
    plan = plan_for(canon, dtype=dtype)
    for streaming in (False, True):
        got = plan.project(target, rhs, max_iterations=500, tolerance=1e-6,
                           streaming=streaming, timing=True)
        assert plan.last_timing()["resident"] == (0 if streaming else 1)
        it = to_np(got.iterations)
        np.testing.assert_array_equal(it[crossed], 500)
        np.testing.assert_array_equal(to_np(got.status), want.status)
        if dtype == np.float64:
            np.testing.assert_array_equal(it, want.iterations)


def test_known_answer_no_constraints_identity():
    """Reference tests/test_regression_chambolle_pock.py:88-95."""
    canon = op.Canonical(n=2, me=0, rows=[], coef=[])
    got, _ = _kn(canon, [[0.2, 0.7]], np.zeros((1, 0)))
    np.testing.assert_allclose(to_np(got.y), [[0.2, 0.7]], atol=1e-12)


@pytest.mark.parametrize("seed", [12, 42])
def test_known_answer_coupled_qp(seed):
    """Reference tests/test_regression_cp_bound_presolve.py:56-101 (exact projection instead of OSQP)."""
    from oracle import qp as bf

    rng = np.random.default_rng(seed)
    canon, rhs = _cases.coupled_qp()
    x = rng.normal(size=(1, 3))
    got, want = _kn(canon, x, rhs[None])
    K = canon.dense()
    y_ref = bf.project_bruteforce(x[0], K[:1], rhs[:1], K[1:], rhs[1:])[0]
    np.testing.assert_allclose(to_np(got.y)[0], y_ref, atol=2e-8)
    mult = to_np(got.multipliers)[0]
    np.testing.assert_allclose((to_np(got.y)[0] - x[0]) + K.T @ mult, 0.0, atol=1e-9)
    assert to_np(got.eligible)[0]


@pytest.mark.parametrize("batch", [1, 127, 129, 300])
def test_ragged_batches(batch):
    torch = require_gpu()
    w = workloads.small_random(3, n=30, me=4, mi=10, width=3, batch=batch)
    canon = canonical_from_workload(w)
    rhs = np.tile(w.rhs, (batch, 1))
    cfg = op.Config(max_iterations=150, early_stop=False)
    want = op.solve(canon, w.target, rhs, cfg)
    got = plan_for(canon, dtype=np.float64).project(w.target, rhs, max_iterations=150,
                                                    early_stop=False)
    assert rel_err(to_np(got.y), want.y) <= 1e-10
    np.testing.assert_array_equal(to_np(got.status), want.status)


def _same_nonfinite(got, want, bar, what):
    """NaN and infinite entries in the same places (infinities with the same
    sign); the finite entries within ``bar`` (relative to the largest)."""
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want), err_msg=what)
    inf = np.isinf(want)
    np.testing.assert_array_equal(np.isinf(got), inf, err_msg=what)
    np.testing.assert_array_equal(got[inf], want[inf], err_msg=what)
    fin = np.isfinite(want)
    assert rel_err(got[fin], want[fin]) <= bar, what


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("early_stop", [False, True])
def test_nonfinite_bounds_and_targets(dtype, early_stop):
    """Per-sample bounds with NaN entries (the lanes whose clip propagates NaN,
    kernels.py:133-147's jnp.clip), infinite bounds, a tied box, and NaN and
    infinite targets, in some samples of a batch: the resident kernel (fixed
    and early stop) and the streaming passes each against the oracle.  NaN
    and infinity land in the same places; the other samples keep the parity
    bar and, in fp64, the oracle's iteration counts (a sample with a
    non-finite iterate never passes the stop test)."""
    torch = require_gpu()
    B = 40
    w = workloads.small_random(13, n=48, me=8, mi=20, width=4, batch=B)
    canon = canonical_from_workload(w)
    rhs = np.tile(w.rhs, (B, 1)).astype(dtype)
    target = w.target.astype(dtype).copy()
    pre = _kept(canon, rhs, dtype)
    ksup, kmask = pre.support[pre.rows], pre.mask[pre.rows]
    lower, upper = pre.lower.astype(dtype).copy(), pre.upper.astype(dtype).copy()
    lower[3, 5] = np.nan
    upper[7, 11] = np.nan
    lower[9, :10], upper[9, :10] = -np.inf, np.inf
    lower[20, 7] = upper[20, 7] = 0.3
    target[12, 2] = np.nan
    target[15, 4] = np.inf
    target[18, 6] = -np.inf
    iters, tol = 300, (1e-6 if dtype == np.float64 else 1e-3)
    with np.errstate(invalid="ignore", over="ignore"):
        mg = Margins(lambda safety, tr: ocp.sparse_cp(
            np.ones_like(target), -target, pre.kept_values[0], pre.kept_rhs, ksup, kmask,
            canon.me, lower, upper, accelerated=False, safety=safety, max_iterations=iters,
            tolerance=tol, y0=target, freeze_converged=True, check_stationarity=True,
            norm_bound=True, early_stop=early_stop, trace=tr), dtype)
    want = mg.want
    assert np.isnan(want.y[3]).any() and np.isnan(want.y[12]).any()
    plan = plan_for(canon, dtype=dtype)
    bar = TOL[dtype]
    for streaming in (False, True):
        got = plan.solve(pre.kept_rhs, target, lower, upper, tolerance=tol, max_iterations=iters,
                         early_stop=early_stop, check_every=5, streaming=streaming, timing=True)
        assert plan.last_timing()["resident"] == (0 if streaming else 1)
        what = f"streaming={streaming}"
        print(f"non-finite inputs: {np.dtype(dtype).name} early_stop={early_stop} {what}",
              flush=True)
        it = to_np(got.iterations)
        same = check_counts(it, mg)
        bad = ~np.all(np.isfinite(want.y), axis=1)  # samples with a non-finite iterate
        assert np.all(it[bad] == iters), what
        y, d = to_np(got.y), to_np(got.dual)
        _same_nonfinite(y[same], want.y[same], bar, what)
        _same_nonfinite(d[same], want.dual[same], bar, what)
        np.testing.assert_array_equal(to_np(got.converged)[same], want.converged[same])
        # tied box: the variable sits on it
        assert np.all(y[20, 7] == dtype(0.3)), what


def test_invalid_arguments_raise():
    torch = require_gpu()
    from purin_amd._lib import PurinError

    canon = _cases.sum_equals_b_u_nonneg()
    plan = plan_for(canon, dtype=np.float64)
    with pytest.raises(ValueError):
        plan.project(np.zeros((2, 3)), np.zeros((2, 2)))
    with pytest.raises(PurinError):
        plan.project(np.zeros((1, 2)), np.zeros((1, 2)), max_iterations=0)


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("accelerated", [False, True])
def test_resident_kernel_matches_streaming_and_oracle(dtype, accelerated):
    """The on-chip resident kernel (fixed iterations) against the streaming passes and the oracle.

    Sizes cover every slot count of the resident schedule (1, 2, 4, 8 per thread).
    """
    torch = require_gpu()
    for n, me, mi, width, B in ((48, 8, 20, 4, 37), (700, 100, 300, 5, 64), (1500, 300, 700, 6, 40),
                                (4096, 1024, 2048, 8, 16)):
        w = workloads.small_random(7 + n, n=n, me=me, mi=mi, width=width, batch=B,
                                   accelerated=accelerated)
        canon = canonical_from_workload(w)
        rhs = np.tile(w.rhs, (B, 1)).astype(dtype)
        target = w.target.astype(dtype)
        plan = plan_for(canon, dtype=dtype, accelerated=accelerated)
        iters = 150
        res = plan.project(target, rhs, max_iterations=iters, early_stop=False, timing=True)
        assert plan.last_timing()["resident"] == 1, n
        st = plan.project(target, rhs, max_iterations=iters, early_stop=False, streaming=True,
                          timing=True)
        assert plan.last_timing()["resident"] == 0
        bar = TOL[dtype]
        assert rel_err(to_np(res.y), to_np(st.y)) <= bar / 10
        assert rel_err(to_np(res.multipliers), to_np(st.multipliers)) <= bar
        np.testing.assert_array_equal(to_np(res.status), to_np(st.status))
        sub = slice(0, 6)
        cfg = op.Config(accelerated=accelerated, max_iterations=iters, early_stop=False)
        want = op.solve(canon, target[sub], rhs[sub], cfg, dtype=dtype)
        assert rel_err(to_np(res.y)[sub], want.y) <= bar, n
        np.testing.assert_array_equal(to_np(res.status)[sub], want.status)


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_resident_random_shapes(dtype):
    """Fourteen shapes drawn from a fixed seed over the resident kernel's range:
    n and m from 1 to 4096 (one to four row and column slots, up to the
    largest tile), no general rows at all, ragged rows of 2 to 12 entries
    (columns of width 0, chunks shared by two slots), batches that leave the
    last tile partly empty; fixed iterations (with bounds shared by the
    samples and scaled per sample) and early stop against the streaming
    passes on the whole batch (fp64 counts identical)."""
    require_gpu()
    rng = np.random.default_rng(2024)
    shapes = [(1, 0, 0), (3, 1, 1), (4096, 0, 0)]
    while len(shapes) < 14:
        n = int(rng.integers(2, 4097))
        m = int(rng.integers(1, 4097))
        me = int(rng.integers(0, m + 1)) // 3
        shapes.append((n, me, m - me))
    bar = TOL[dtype]
    for k, (n, me, mi) in enumerate(shapes):
        B = int(rng.integers(1, 300))
        wmax = min(12, n)
        wmin = min(2, wmax)
        w = workloads.ragged_rows(400 + k, n=n, me=me, mi=mi, wmin=wmin, wmax=wmax, batch=B,
                                  accelerated=bool(k % 2))
        canon = canonical_from_workload(w)
        rhs = np.tile(w.rhs, (B, 1)).astype(dtype)
        target = w.target.astype(dtype)
        plan = plan_for(canon, dtype=dtype, accelerated=bool(k % 2))
        print(f"random shape {k}: n={n} me={me} mi={mi} B={B} {np.dtype(dtype).name}",
              flush=True)
        kw = dict(max_iterations=60, early_stop=False, timing=True)
        res = plan.project(target, rhs, **kw)
        assert plan.last_timing()["resident"] == 1, (k, n, me, mi)
        st = plan.project(target, rhs, streaming=True, **kw)
        assert rel_err(to_np(res.y), to_np(st.y)) <= bar / 10, (k, n, me, mi)
        assert rel_err(to_np(res.multipliers), to_np(st.multipliers)) <= bar, (k, n, me, mi)
        np.testing.assert_array_equal(to_np(res.status), to_np(st.status))
        # bounds scaled per sample (the last 2n rows: y <= 1, -y <= 1); the
        # kernel holds the leading column slots' bounds that fit in LDS
        f = np.random.default_rng(600 + k).uniform(0.5, 1.5, B)
        rv = np.tile(w.rhs, (B, 1))
        rv[:, -2 * n:] *= f[:, None]
        rv = rv.astype(dtype)
        rp = plan.project(target, rv, **kw)
        assert plan.last_timing()["resident"] == 1, (k, n, me, mi)
        sp = plan.project(target, rv, streaming=True, **kw)
        assert rel_err(to_np(rp.y), to_np(sp.y)) <= bar / 10, (k, n, me, mi)
        assert rel_err(to_np(rp.multipliers), to_np(sp.multipliers)) <= bar, (k, n, me, mi)
        kw = dict(max_iterations=300, early_stop=True, tolerance=1e-3, timing=True)
        re_ = plan.project(target, rhs, **kw)
        assert plan.last_timing()["resident"] == 1, (k, n, me, mi)
        se = plan.project(target, rhs, streaming=True, **kw)
        it_r, it_s = to_np(re_.iterations), to_np(se.iterations)
        same = it_r == it_s
        if dtype == np.float64:
            np.testing.assert_array_equal(it_r, it_s)
        assert rel_err(to_np(re_.y)[same], to_np(se.y)[same]) <= bar, (k, n, me, mi)
        np.testing.assert_array_equal(to_np(re_.status)[same], to_np(se.status)[same])


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_resident_largest_tile(dtype):
    """The largest problem the resident kernels take: n = m = 4096, four row
    and four column slots per thread, a 131,104-byte LDS image (150,576 bytes
    in the early-stop kernel with shared bounds, which keeps K y of one row
    slot in LDS; with per-sample bounds it keeps K y in registers, and no
    slot of bounds fits beside the image; either re-reads targets and
    right-hand sides each iteration).  Fixed iterations
    with per-sample and with shared bounds (bit-identical), against the
    streaming passes and, on two samples, the oracle; early stop in fp64 with
    the streaming passes' iteration counts."""
    require_gpu()
    n, me, mi, B = 4096, 1024, 3072, 10
    w = workloads.small_random(91, n=n, me=me, mi=mi, width=6, batch=B, accelerated=True)
    canon = canonical_from_workload(w)
    rhs = np.tile(w.rhs, (B, 1)).astype(dtype)
    target = w.target.astype(dtype)
    plan = plan_for(canon, dtype=dtype, accelerated=True)
    info = plan.info
    assert info.resident_row_slots == 4096 and info.resident_col_slots == 4096
    bar = TOL[dtype]
    iters = 120
    res = plan.project(target, rhs, max_iterations=iters, early_stop=False, timing=True)
    assert plan.last_timing()["resident"] == 1
    st = plan.project(target, rhs, max_iterations=iters, early_stop=False, streaming=True)
    assert rel_err(to_np(res.y), to_np(st.y)) <= bar / 10
    assert rel_err(to_np(res.multipliers), to_np(st.multipliers)) <= bar
    np.testing.assert_array_equal(to_np(res.status), to_np(st.status))
    sh = plan.project(target, rhs, max_iterations=iters, early_stop=False, shared_bounds=True)
    np.testing.assert_array_equal(to_np(sh.y), to_np(res.y))
    sub = slice(0, 2)
    cfg = op.Config(accelerated=True, max_iterations=iters, early_stop=False)
    want = op.solve(canon, target[sub], rhs[sub], cfg, dtype=dtype)
    assert rel_err(to_np(res.y)[sub], want.y) <= bar
    np.testing.assert_array_equal(to_np(res.status)[sub], want.status)
    if dtype == np.float64:
        # this problem converges slowly: at tolerance 0.3 the samples stop at
        # different iterations (about 430-580), so tiles freeze samples one by one
        kw = dict(max_iterations=700, early_stop=True, tolerance=0.3)
        for shared in (False, True):
            re_ = plan.project(target, rhs, timing=True, shared_bounds=shared, **kw)
            assert plan.last_timing()["resident"] == 1
            se = plan.project(target, rhs, streaming=True, shared_bounds=shared, **kw)
            it = to_np(re_.iterations)
            np.testing.assert_array_equal(it, to_np(se.iterations))
            np.testing.assert_array_equal(to_np(re_.status), to_np(se.status))
            assert rel_err(to_np(re_.y), to_np(se.y)) <= bar
        assert np.all(it < kw["max_iterations"]) and len(np.unique(it)) > 2


# (n, me, mi, dtype, the column slots whose per-sample bounds the fixed-iteration
# resident kernel holds in LDS: what fits of 160 KB beside the image, at most
# the column slot count)
LDS_BOUNDS = ((1000, 100, 200, np.float64, 1), (2000, 200, 400, np.float64, 2),
              (3000, 300, 500, np.float64, 3), (4096, 200, 400, np.float64, 2),
              (4096, 1024, 2048, np.float64, 1), (3000, 300, 500, np.float32, 3),
              (800, 100, 200, np.float32, 1))


def _lds_bound_slots(info, dtype):
    """The kernel's rule, restated: 16-byte entries (n + 1 + m + 1), or two
    planes of 32,800 bytes for 8-sample fp32 tiles; a slot's bounds take
    2 x 1024 x 16 bytes per 16 bytes of tile samples."""
    samples = info.resident_tile_samples
    vb = samples * np.dtype(dtype).itemsize
    image = 2 * 32800 if samples == 8 else (info.n + 1 + info.kept_rows + 1) * 16
    return min(info.resident_col_slots // 1024, (160 * 1024 - image) // (2 * 1024 * vb))


@pytest.mark.parametrize("case", range(len(LDS_BOUNDS)))
def test_resident_per_sample_bounds_held_in_lds(case):
    """Per-sample bounds with one to three column slots held in LDS by the
    fixed-iteration resident kernel (the rest read from memory): bounds equal
    in every sample give the shared-bounds bits; bounds scaled per sample
    (upper f_b, lower -f_b, f_b in [0.5, 1.5]) match the streaming passes on
    the whole batch and the oracle on two samples, at the parity bars; early
    stop (the early-stop kernel holds the bounds in place of K y) matches the
    streaming passes' counts (identical in fp64) and iterates."""
    require_gpu()
    n, me, mi, dtype, want_slots = LDS_BOUNDS[case]
    B = 37
    w = workloads.small_random(700 + case, n=n, me=me, mi=mi, width=5, batch=B,
                               accelerated=True)
    canon = canonical_from_workload(w)
    plan = plan_for(canon, dtype=dtype, accelerated=True)
    assert _lds_bound_slots(plan.info, dtype) == want_slots, case
    bar = TOL[dtype]
    target = w.target.astype(dtype)
    rhs = np.tile(w.rhs, (B, 1)).astype(dtype)
    kw = dict(max_iterations=150, early_stop=False)
    print(f"bounds in LDS: n={n} m={me + mi} {np.dtype(dtype).name} slots={want_slots}",
          flush=True)
    ps = plan.project(target, rhs, timing=True, **kw)
    assert plan.last_timing()["resident"] == 1
    sh = plan.project(target, rhs, shared_bounds=True, **kw)
    np.testing.assert_array_equal(to_np(ps.y), to_np(sh.y))
    np.testing.assert_array_equal(to_np(ps.multipliers), to_np(sh.multipliers))
    # the last 2n rows are the bound rows (y <= 1, then -y <= 1)
    f = np.random.default_rng(case).uniform(0.5, 1.5, B)
    rhs_v = np.tile(w.rhs, (B, 1))
    rhs_v[:, -2 * n:] *= f[:, None]
    rhs_v = rhs_v.astype(dtype)
    got = plan.project(target, rhs_v, timing=True, **kw)
    assert plan.last_timing()["resident"] == 1
    st = plan.project(target, rhs_v, streaming=True, **kw)
    assert rel_err(to_np(got.y), to_np(st.y)) <= bar / 10, case
    assert rel_err(to_np(got.multipliers), to_np(st.multipliers)) <= bar, case
    np.testing.assert_array_equal(to_np(got.status), to_np(st.status))
    assert not np.array_equal(to_np(got.y), to_np(ps.y))  # the bounds bind differently
    sub = slice(0, 2)
    cfg = op.Config(accelerated=True, max_iterations=150, early_stop=False)
    want = op.solve(canon, target[sub], rhs_v[sub], cfg, dtype=dtype)
    assert rel_err(to_np(got.y)[sub], want.y) <= bar, case
    np.testing.assert_array_equal(to_np(got.status)[sub], want.status)
    # the early-stop kernel holds the same slots' bounds in place of K y
    ke = dict(max_iterations=400, early_stop=True, tolerance=1e-3)
    ge = plan.project(target, rhs_v, timing=True, **ke)
    assert plan.last_timing()["resident"] == 1
    se = plan.project(target, rhs_v, streaming=True, **ke)
    it_g, it_s = to_np(ge.iterations), to_np(se.iterations)
    same = it_g == it_s
    if dtype == np.float64:
        np.testing.assert_array_equal(it_g, it_s)
    assert same.mean() >= 0.9, case
    assert rel_err(to_np(ge.y)[same], to_np(se.y)[same]) <= bar, case
    np.testing.assert_array_equal(to_np(ge.status)[same], to_np(se.status)[same])


# ragged rows: (n, me, mi, wmin, wmax, B).  The resident schedule packs each
# wavefront's slots back to back, so a chunk may hold the end of one slot and
# the start of the next: these shapes give split chunks in the row pass (3 and
# 4 row slots of unequal widths) and in the column pass, and slots narrower
# than a chunk (mostly empty columns: widths 0-2)
RAGGED = ((2500, 700, 1800, 2, 11, 20), (4000, 100, 400, 2, 5, 9), (1000, 1200, 2800, 2, 9, 33))


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("accelerated", [False, True])
def test_resident_packed_slots_ragged_rows(dtype, accelerated):
    """The resident kernels on rows and columns of unequal lengths (packed slots,
    chunks shared by two slots) against the streaming passes and the oracle, in
    fixed-iteration and early-stop mode."""
    require_gpu()
    for k, (n, me, mi, wmin, wmax, B) in enumerate(RAGGED):
        w = workloads.ragged_rows(50 + k, n=n, me=me, mi=mi, wmin=wmin, wmax=wmax, batch=B,
                                  accelerated=accelerated)
        canon = canonical_from_workload(w)
        rhs = np.tile(w.rhs, (B, 1)).astype(dtype)
        target = w.target.astype(dtype)
        plan = plan_for(canon, dtype=dtype, accelerated=accelerated)
        bar = TOL[dtype]
        iters = 150
        res = plan.project(target, rhs, max_iterations=iters, early_stop=False, timing=True)
        assert plan.last_timing()["resident"] == 1, n
        st = plan.project(target, rhs, max_iterations=iters, early_stop=False, streaming=True)
        assert rel_err(to_np(res.y), to_np(st.y)) <= bar / 10, n
        assert rel_err(to_np(res.multipliers), to_np(st.multipliers)) <= bar, n
        np.testing.assert_array_equal(to_np(res.status), to_np(st.status))
        # the shared-bounds kernel (bounds from registers) gives the same bits
        sh = plan.project(target, rhs, max_iterations=iters, early_stop=False,
                          shared_bounds=True)
        np.testing.assert_array_equal(to_np(sh.y), to_np(res.y))
        sub = slice(0, 2)
        cfg = op.Config(accelerated=accelerated, max_iterations=iters, early_stop=False)
        want = op.solve(canon, target[sub], rhs[sub], cfg, dtype=dtype)
        assert rel_err(to_np(res.y)[sub], want.y) <= bar, n
        np.testing.assert_array_equal(to_np(res.status)[sub], want.status)
        if dtype == np.float64:  # early stop: identical iteration counts in fp64
            kw = dict(max_iterations=600, early_stop=True, tolerance=1e-5 if accelerated else 1e-4)
            re_ = plan.project(target, rhs, timing=True, **kw)
            assert plan.last_timing()["resident"] == 1, n
            se = plan.project(target, rhs, streaming=True, **kw)
            np.testing.assert_array_equal(to_np(re_.iterations), to_np(se.iterations))
            np.testing.assert_array_equal(to_np(re_.status), to_np(se.status))
            assert rel_err(to_np(re_.y), to_np(se.y)) <= bar, n


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("accelerated", [False, True])
def test_resident_early_stop_matches_streaming_and_oracle(dtype, accelerated):
    """Early stop on the resident kernel (each workgroup stops when its samples
    are accepted; accepted samples keep their state and count) against the
    streaming passes and the oracle.  The resident early-stop kernel forms
    K ybar from the last two residual sweeps ((1 + theta) K y - theta K y_prev)
    instead of gathering ybar, and its stop test sums the objective terms in
    another fixed order, so its iterates differ from the streaming passes' by
    rounding: same-count samples agree to the parity bar; fp64 counts are
    identical; in fp32 a sample whose margin sits on the tolerance may stop
    one iteration apart (at most 1 in 10).

    Oracle leg, fp64 and fp32: on the first samples of each batch the
    resident kernel's counts are the oracle's under the rule of
    tests/_margins.py (identical in fp64; in fp32 a different count only at a
    borderline stop), same-count iterates at the parity bar and statuses
    equal; the others within the oracle's own spread under a 1e-6 change of
    the steps (accelerated fp32 moves some stops by tens of iterations)."""
    torch = require_gpu()
    tol = (1e-6 if dtype == np.float64 else 1e-3) if not accelerated else 1e-4
    # oracle samples per size (the NumPy oracle's per-iteration diagnostics
    # dominate the test's time at the larger sizes)
    n_oracle = {48: 8, 700: 6, 1500: 4, 4096: 2}
    stopped = 0
    for n, me, mi, width, B in ((48, 8, 20, 4, 37), (700, 100, 300, 5, 64), (1500, 300, 700, 6, 40),
                                (4096, 1024, 2048, 8, 16)):
        w = workloads.small_random(3 + n, n=n, me=me, mi=mi, width=width, batch=B,
                                   accelerated=accelerated)
        canon = canonical_from_workload(w)
        rhs = np.tile(w.rhs, (B, 1)).astype(dtype)
        target = w.target.astype(dtype)
        plan = plan_for(canon, dtype=dtype, accelerated=accelerated)
        kw = dict(max_iterations=2000, early_stop=True, tolerance=tol, timing=True)
        res = plan.project(target, rhs, **kw)
        assert plan.last_timing()["resident"] == 1, n
        st = plan.project(target, rhs, streaming=True, **kw)
        assert plan.last_timing()["resident"] == 0
        it_r, it_s = to_np(res.iterations), to_np(st.iterations)
        same = it_r == it_s
        if dtype == np.float64:
            np.testing.assert_array_equal(it_r, it_s)
        elif not accelerated:
            assert (~same).sum() * 10 <= B, (n, it_r[~same], it_s[~same])
            assert np.all(np.abs(it_r - it_s) <= 1)
        # accelerated fp32: the stop iteration itself moves by up to a few hundred
        # iterations under rounding-level changes of the iterate (measured: the
        # streaming passes and the oracle differ as much at n = 48), so the counts
        # are not compared there.  Samples stopped at the same iteration agree to
        # the parity bar; two points that each passed the stop test at tolerance
        # tol but at different iterations agree to that tolerance's scale, 2 tol
        yr, ys = to_np(res.y), to_np(st.y)
        assert rel_err(yr[same], ys[same]) <= TOL[dtype]
        assert rel_err(yr, ys) <= (2 * tol if dtype == np.float32 and accelerated else TOL[dtype])
        assert rel_err(to_np(res.multipliers)[same], to_np(st.multipliers)[same]) <= TOL[dtype]
        if dtype == np.float64 or not accelerated:
            np.testing.assert_array_equal(to_np(res.status)[same], to_np(st.status)[same])
        stopped += int(np.sum(it_r < kw["max_iterations"]))
        sub = np.arange(n_oracle[n])
        cfg = op.Config(accelerated=accelerated, max_iterations=kw["max_iterations"],
                        tolerance=tol)
        print(f"n={n} {np.dtype(dtype).name} accelerated={accelerated}: oracle on "
              f"{sub.size} samples", flush=True)
        mg = Margins(lambda safety, tr: op.solve(canon, target[sub], rhs[sub],
                                                 replace(cfg, safety=safety), dtype=dtype,
                                                 trace=tr), dtype)
        print(f"  counts gpu {it_r[sub].tolist()} oracle {mg.want.iterations.tolist()}",
              flush=True)
        same_o = check_counts(it_r, mg, samples=sub)
        check_iterates(to_np(res.y), mg, same_o, TOL[dtype], samples=sub)
        np.testing.assert_array_equal(to_np(res.status)[sub][same_o], mg.want.status[same_o])
    assert stopped > 0  # the stop test fired


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("accelerated", [False, True])
@pytest.mark.parametrize("early_stop", [False, True])
def test_streaming_linear_kybar_matches_oracle(dtype, accelerated, early_stop):
    """Wide problems (n > 2m): the streaming passes form K ybar as
    (1 + theta) K y - theta K y_prev (kernels.py:149 applied under K) instead of
    storing ybar; with the stop test the row pass takes K y from the residual
    pass and gathers nothing.  Against the oracle (which forms ybar and
    gathers it) at the parity bar, with the oracle's iteration counts and
    statuses in fp64, and against the resident kernel on the same inputs."""
    torch = require_gpu()
    bar = TOL[dtype]
    # tolerances at which the oracle stops these samples within the limit
    # (fixed step: all of them at both sizes; accelerated: the n = 200 ones)
    tol = 1e-3 if accelerated else 1e-4
    stopped = 0
    for n, me, mi, width, B in ((200, 20, 60, 4, 37), (3000, 300, 900, 6, 40)):
        w = workloads.small_random(21 + n, n=n, me=me, mi=mi, width=width, batch=B,
                                   accelerated=accelerated, target_sd=0.5)
        canon = canonical_from_workload(w)
        rhs = np.tile(w.rhs, (B, 1)).astype(dtype)
        target = w.target.astype(dtype)
        plan = plan_for(canon, dtype=dtype, accelerated=accelerated)
        iters = 400
        kw = dict(max_iterations=iters, early_stop=early_stop, tolerance=tol)
        st = plan.project(target, rhs, streaming=True, timing=True, **kw)
        t = plan.last_timing()
        assert t["resident"] == 0 and t["linear_kybar"] == 1, n
        res = plan.project(target, rhs, timing=True, **kw)
        assert plan.last_timing()["resident"] == 1
        sub = slice(0, 6)
        cfg = op.Config(accelerated=accelerated, max_iterations=iters, early_stop=early_stop,
                        tolerance=tol)
        want = op.solve(canon, target[sub], rhs[sub], cfg, dtype=dtype)
        assert rel_err(to_np(st.y)[sub], want.y) <= bar, n
        if dtype == np.float64:
            np.testing.assert_array_equal(to_np(st.iterations)[sub], want.iterations)
            np.testing.assert_array_equal(to_np(st.status)[sub], want.status)
            np.testing.assert_array_equal(to_np(st.iterations), to_np(res.iterations))
        assert rel_err(to_np(st.y), to_np(res.y)) <= bar
        stopped += int(np.sum(to_np(st.iterations) < iters))
    if early_stop:
        assert stopped > 0  # the stop test fired


def test_streaming_early_stop_two_pass_fold():
    """The streaming passes' stop test at B = 256 (4 blocks of 64 samples),
    where the chunk partials are folded in two passes (every 16th chunk per
    block of the first pass, then the 16 partials), on a problem whose
    fixed-iteration column pass takes quarter-wavefront tiles (m = 4500 kept
    rows).  Against the oracle's early stop on samples from both ends of the
    batch: identical iteration counts and statuses, y at the fp64 bar."""
    require_gpu()
    B = 256
    w = workloads.small_random(77, n=10000, me=1500, mi=3000, width=4, batch=B,
                               accelerated=True, target_sd=0.5)
    canon = canonical_from_workload(w)
    rhs = np.tile(w.rhs, (B, 1))
    target = np.ascontiguousarray(w.target, np.float64)
    plan = plan_for(canon, dtype=np.float64, accelerated=True)
    kw = dict(max_iterations=800, early_stop=True, tolerance=1e-2)
    got = plan.project(target, rhs, timing=True, **kw)
    t = plan.last_timing()
    assert t["resident"] == 0
    pick = [0, 1, B - 2, B - 1]
    cfg = op.Config(accelerated=True, max_iterations=800, early_stop=True, tolerance=1e-2)
    want = op.solve(canon, target[pick], rhs[pick], cfg, dtype=np.float64)
    np.testing.assert_array_equal(to_np(got.iterations)[pick], want.iterations)
    np.testing.assert_array_equal(to_np(got.status)[pick], want.status)
    assert rel_err(to_np(got.y)[pick], want.y) <= TOL[np.float64]
