"""Parity at the benchmark configurations' full sizes.

At these sizes the oracle cannot run the whole batch in seconds, so each test
checks (1) a few samples from both ends of the batch against the checker
(the C restatement of the CP loop, bit-equal to the NumPy oracle, or the NumPy
adjoint), and (2) a size-independent property: samples are independent, so
the first samples projected alone give bit-identical results to the same
samples inside the full batch.
"""

import numpy as np
import pytest

from oracle import cloop
from oracle import projection as op
from purin_amd import workloads
from tests._gpu import rel_err, require_gpu, to_np

pytestmark = pytest.mark.gpu

PICK = np.array([0, 1, 2, -3, -2, -1])


@pytest.fixture(scope="module", autouse=True)
def checker_library():
    cloop.load()


def full_plan(w):
    import torch

    from purin_amd.plan import Plan

    values, root = w.data, None
    if w.metric is not None:
        root = np.sqrt(np.asarray(w.metric, np.float64))
        values = w.data / root[w.indices]
    p = Plan(w.n, w.me, w.rows_total - w.me, w.indptr, w.indices, values,
             dtype=torch.float64 if w.dtype == np.float64 else torch.float32,
             accelerated=w.accelerated, device="cuda")
    if root is not None:
        p.set_metric(root)
    return p, values, root


class Checked:
    """The C loop's fixed-iteration state on a few samples, and the oracle's
    recovery of the projection outputs from it (bounds.py:247-317)."""

    def __init__(self, w, values, root, samples):
        from oracle import cp as ocp

        rows = [list(w.indices[w.indptr[i]:w.indptr[i + 1]]) for i in range(w.rows_total)]
        coef = [list(values[w.indptr[i]:w.indptr[i + 1]]) for i in range(w.rows_total)]
        self.canon = op.Canonical(n=w.n, me=w.me, rows=rows, coef=coef)
        dt = np.dtype(w.dtype)
        target = np.asarray(w.target[samples], dt)
        if root is not None:  # the plan's variables z = sqrt(D) y (metric.py:102-108)
            target = target * root.astype(dt)
        self.target = target
        self.rhs = np.tile(w.rhs, (len(samples), 1)).astype(dt)
        self.cfg = op.Config(accelerated=w.accelerated, max_iterations=w.iterations,
                             early_stop=False)
        self.y, self.d, _ = cloop.run(cloop.prepare(self.canon, target, self.rhs, self.cfg, dt),
                                      w.iterations, w.accelerated, threads=8)
        # final diagnostics (kernels.py:291-305) and recovery, as oracle.cp.sparse_cp and
        # oracle.projection.solve finish a fixed-iteration run
        pre = op.presolve(self.canon, self.rhs, self.cfg, dt)
        self.pre = pre
        ksup, kmask = pre.support[pre.rows], pre.mask[pre.rows]
        mv, tmv = ocp.operators(pre.kept_values[0], ksup, kmask, w.n)
        q, c = np.ones_like(target), -target
        res, gap = ocp.diagnostics(self.y, self.d, q, c, pre.kept_rhs, pre.lower, pre.upper, mv,
                                   tmv, w.me)
        stat = ocp.stationarity(self.y, self.d, q, c, pre.lower, pre.upper, tmv)
        finite = (np.all(np.isfinite(self.y), axis=1) & np.all(np.isfinite(self.d), axis=1)
                  & np.isfinite(gap) & np.isfinite(res))
        conv = finite & (res <= pre.tolerance) & (gap <= pre.tolerance) & (stat <= pre.tolerance)
        iters = np.full(len(samples), w.iterations, np.int32)
        out = ocp.CPOutput(self.y, self.d, iters, np.maximum(res, stat), gap,
                           conv & pre.feasible)
        self.rec = op.recover(self.canon, pre, out, target, self.rhs, self.cfg)
        self.multipliers = np.concatenate((self.rec.multipliers_eq, self.rec.multipliers_ineq),
                                          axis=1)


def checker_y(w, values, root, samples):
    """y of the C loop for ``samples`` (in the metric's variables when there is one)."""
    return Checked(w, values, root, samples).y


def spread(B, k):
    """Both ends of the batch and ``k`` samples spread over it."""
    return np.unique(np.r_[[0, 1, 2, B - 3, B - 2, B - 1],
                           np.linspace(0, B - 1, k).astype(int)])


def test_full_size_duals_and_active_sets():
    """Kept-row duals, recovered multipliers, slacks, status and the active-set
    masks at the full benchmark sizes, against the checker on samples spread
    over the batch (configs 2, 3, 4: fp64 1e-10 and fp32 1e-4 on values; masks
    identical).  The masks are the reference's: ``y == lower`` and
    ``y == upper`` as the dual recovery tests them (bounds.py:252-261), in the
    plan's variables (config 3's metric variables z = sqrt(D) y), ``d_I > 0`` on
    the kept inequality rows (kernels.py:133-136), and positive recovered bound
    multipliers.  ``solve`` gives the kept-row duals and z directly;
    ``project`` the multipliers (original units), slacks and status."""
    import torch

    require_gpu()
    for config, k in ((2, 26), (3, 10), (4, 58)):
        w = {2: workloads.config2, 3: workloads.config3, 4: workloads.config4}[config]()
        B = w.target.shape[0]
        samples = spread(B, k)
        p, values, root = full_plan(w)
        dt = np.dtype(w.dtype)
        bar = 1e-10 if dt == np.float64 else 1e-4
        print(f"config{config}: B={B} n={w.n} iterations={w.iterations}, "
              f"{len(samples)} checked samples", flush=True)
        ck = Checked(w, values, root, samples)
        pre = ck.pre
        rhs = np.tile(w.rhs, (B, 1)).astype(dt)
        kw = dict(max_iterations=w.iterations, early_stop=False, shared_bounds=True)
        # the inner solve in the plan's variables and scaled units
        target_z = w.target.astype(dt) * (root.astype(dt) if root is not None else 1)
        o = p.solve(np.tile(pre.kept_rhs[0], (B, 1)), target_z, pre.lower[0], pre.upper[0], **kw)
        yz, d = to_np(o.y)[samples], to_np(o.dual)[samples]
        del o
        me = w.me
        lo, hi = pre.lower, pre.upper
        print(f"  solve: y {rel_err(yz, ck.y):.2e} dual {rel_err(d, ck.d):.2e}; "
              f"at lower {int((ck.y == lo).sum())} (gpu {int((yz == lo).sum())}), at upper "
              f"{int((ck.y == hi).sum())} (gpu {int((yz == hi).sum())}), active inequalities "
              f"{int((ck.d[:, me:] > 0).sum())} (gpu {int((d[:, me:] > 0).sum())})", flush=True)
        # the whole projection
        out = p.project(w.target, rhs, **kw)
        y = to_np(out.y)[samples]
        mult = to_np(out.multipliers)[samples]
        slacks = to_np(out.slacks)[samples]
        status = to_np(out.status)[samples]
        residual = to_np(out.residual)[samples]
        del out
        kept, bnd = pre.rows, pre.bounds
        print(f"  project: y {rel_err(y * (root if root is not None else 1), ck.y):.2e} "
              f"kept multipliers {rel_err(mult[:, kept], ck.multipliers[:, kept]):.2e} "
              f"bound multipliers {rel_err(mult[:, bnd], ck.multipliers[:, bnd]):.2e} "
              f"slacks {rel_err(slacks, ck.rec.slacks):.2e} status {np.unique(status)} "
              f"residual {residual.min():.3e}..{residual.max():.3e} vs "
              f"{ck.rec.residual_inf_norm.min():.3e}..{ck.rec.residual_inf_norm.max():.3e}, "
              f"positive bound multipliers {int((ck.multipliers[:, bnd] > 0).sum())} "
              f"(gpu {int((mult[:, bnd] > 0).sum())})", flush=True)
        # values at the parity bar
        assert rel_err(yz, ck.y) <= bar
        assert rel_err(d, ck.d) <= bar
        assert rel_err(mult[:, kept], ck.multipliers[:, kept]) <= bar
        if len(bnd):
            assert rel_err(mult[:, bnd], ck.multipliers[:, bnd]) <= bar
        assert rel_err(slacks, ck.rec.slacks) <= bar
        np.testing.assert_array_equal(status, ck.rec.status)
        # the original-unit residual; with a metric it is the z-space residual times
        # max(1, sqrt(max D)) (metric.py:161-165)
        factor = max(1.0, float(np.max(root))) if root is not None else 1.0
        np.testing.assert_allclose(residual, ck.rec.residual_inf_norm * factor,
                                   rtol=1e-8 if dt == np.float64 else 1e-3)
        # the active sets, identical
        np.testing.assert_array_equal(yz == lo, ck.y == lo)
        np.testing.assert_array_equal(yz == hi, ck.y == hi)
        np.testing.assert_array_equal(d[:, me:] > 0, ck.d[:, me:] > 0)
        np.testing.assert_array_equal(mult[:, bnd] > 0, ck.multipliers[:, bnd] > 0)
        # the non-vacuous part: bounds are attained and inequalities active
        assert (ck.y == lo).any() or (ck.y == hi).any()
        assert config == 3 or (ck.d[:, me:] > 0).any()
        del p
        torch.cuda.empty_cache()


def test_full_size_resident_and_streaming_agree():
    """config2: the on-chip kernel and the streaming passes on the whole batch."""
    require_gpu()
    w = workloads.config2()
    B = w.target.shape[0]
    p, _, _ = full_plan(w)
    rhs = np.tile(w.rhs, (B, 1))
    kw = dict(max_iterations=w.iterations, early_stop=False, shared_bounds=True)
    res = p.project(w.target, rhs, timing=True, **kw)
    assert p.last_timing()["resident"] == 1
    st = p.project(w.target, rhs, streaming=True, **kw)
    assert rel_err(to_np(res.y), to_np(st.y)) <= 1e-11
    assert rel_err(to_np(res.multipliers), to_np(st.multipliers)) <= 1e-10
    np.testing.assert_array_equal(to_np(res.status), to_np(st.status))
    ya, yb = to_np(res.y), to_np(st.y)
    np.testing.assert_array_equal(ya == -1.0, yb == -1.0)
    np.testing.assert_array_equal(ya == 1.0, yb == 1.0)


C_BOUND = 50.0  # VJP distance from the converged one per unit GMRES residual (test_oracle_vjp_steps.py)


def _row_rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.max(np.abs(a - b), axis=1) / np.max(np.abs(b), axis=1)


def test_full_size_adjoint_at_the_same_state():
    """config5: the VJP of the full 1024-sample batch (eligibility forced at the
    2000-iteration state) against the oracle's adjoint linearised at the GPU's
    own state, on 16 samples spread over the batch.

    * default GMRES (tolerance 1e-9, restart 30, 100 steps): every sample stops
      at the step limit with a residual of about 1e-5; the iterate is accepted
      (adjoint_tolerance = 1, else both sides return zero gradients) and held
      to the oracle's at 1e-8, per-sample Arnoldi steps and info codes equal,
      and within C_BOUND times the GMRES residual of the converged VJP: the
      bound that holds whatever the adjoint's tau and sigma (the reference's
      start vector cannot be reproduced here);
    * tolerance 1e-4: samples stop at different steps (about 88 to 100); the
      counts equal the oracle's;
    * tolerance 1e-14 (1000 steps, converged): held to 1e-10.
    """
    import torch

    from oracle import adjoint as oadj

    require_gpu()
    w = workloads.config5()
    B = w.target.shape[0]
    p, _, _ = full_plan(w)
    cfg = op.Config(accelerated=True, max_iterations=w.iterations, early_stop=False)
    one = op.Canonical(n=w.n, me=w.me, rows=w.rows(), coef=w.coefs())
    pre = op.presolve(one, w.rhs[None, :], cfg, np.float64)
    rhs_k = np.tile(pre.kept_rhs, (B, 1))
    o, saved = p.solve(rhs_k, w.target, pre.lower[0], pre.upper[0], max_iterations=w.iterations,
                       early_stop=False, shared_bounds=True, save=True)
    y, d = to_np(o.y), to_np(o.dual)
    ksup, kmask = pre.support[pre.rows], pre.mask[pre.rows]
    sub = np.linspace(0, B - 1, 16).astype(int)

    def oracle(rows, tol, maxit):
        c = op.Config(accelerated=True, max_iterations=w.iterations, early_stop=False,
                      gmres_tolerance=tol, gmres_max_iterations=maxit, adjoint_tolerance=1.0)
        k = len(rows)
        return oadj.adjoint(pre.kept_values[0], ksup, kmask, w.me, y[rows], d[rows],
                            np.ones(k, bool), w.target[rows], rhs_k[rows],
                            np.broadcast_to(pre.lower[0], (k, w.n)),
                            np.broadcast_to(pre.upper[0], (k, w.n)), w.cotangent[rows], c)

    def gpu(tol, maxit):
        a = p.adjoint(saved, w.target, rhs_k, w.cotangent, force_eligible=True, rhs_rows=p.m,
                      tolerance=tol, max_iterations=maxit, adjoint_tolerance=1.0)
        steps = to_np(p.last_adjoint_iterations(B))
        torch.cuda.synchronize()
        return a, steps

    # default GMRES: the accepted 100-step iterate
    print("config5 adjoint: default GMRES, 16 samples", flush=True)
    adj, steps = gpu(1e-9, 100)
    want = oracle(sub, 1e-9, 100)
    gscale = np.max(np.abs(w.cotangent[sub]), axis=1)
    gt, gr = to_np(adj.g_target)[sub], to_np(adj.g_rhs)[sub]
    rho = to_np(adj.residual)[sub] / gscale
    rho_o = want.residual / gscale
    four = sub[[0, 5, 10, 15]]
    k4 = np.searchsorted(sub, four)
    print("config5 adjoint: GMRES 1e-14, 4 samples", flush=True)
    conv = oracle(four, 1e-14, 1000)
    adj14, _ = gpu(1e-14, 1000)
    print("config5 adjoint: GMRES 1e-4, 16 samples", flush=True)
    adj6, steps6 = gpu(1e-4, 100)
    want6 = oracle(sub, 1e-4, 100)
    print("default: gpu vs oracle gt", _row_rel(gt, want.g_target), "gr", _row_rel(gr, want.g_rhs),
          "rho", rho, "rho_oracle", rho_o, flush=True)
    print("default vs converged: gpu gt", _row_rel(gt[k4], conv.g_target), "oracle gt",
          _row_rel(want.g_target[k4], conv.g_target), flush=True)
    print("1e-14: gt", _row_rel(to_np(adj14.g_target)[four], conv.g_target), "gr",
          _row_rel(to_np(adj14.g_rhs)[four], conv.g_rhs), "info", to_np(adj14.info)[four],
          conv.info, flush=True)
    print("1e-4: steps", steps6[sub], want6.iterations, "gt",
          _row_rel(to_np(adj6.g_target)[sub], want6.g_target), flush=True)
    # the default leg
    np.testing.assert_array_equal(to_np(adj.info)[sub], want.info)
    np.testing.assert_array_equal(steps[sub], want.iterations)
    assert np.all(to_np(adj.valid)[sub]) and np.all(want.valid)
    assert np.all(rho > 1e-7)  # unconverged: the bounds below are not vacuous
    # both iterates lie within C_BOUND * rho of the converged VJP, so they are
    # within C_BOUND * (rho + rho_oracle) of each other
    assert np.all(_row_rel(gt, want.g_target) <= C_BOUND * (rho + rho_o))
    assert np.all(_row_rel(gr, want.g_rhs) <= C_BOUND * (rho + rho_o))
    assert np.all(_row_rel(gt[k4], conv.g_target) <= C_BOUND * rho[k4])
    assert np.all(_row_rel(gr[k4], conv.g_rhs) <= C_BOUND * rho[k4])
    # converged: the VJP is defined to rounding, and held to 1e-10
    assert np.all(conv.info == 0) and np.all(to_np(adj14.info)[four] == 0)
    assert np.all(_row_rel(to_np(adj14.g_target)[four], conv.g_target) <= 1e-10)
    assert np.all(_row_rel(to_np(adj14.g_rhs)[four], conv.g_rhs) <= 1e-10)
    # per-sample Arnoldi steps where the samples stop at different steps
    assert len(np.unique(want6.iterations)) > 1
    np.testing.assert_array_equal(steps6[sub], want6.iterations)
    np.testing.assert_array_equal(to_np(adj6.info)[sub], want6.info)


def test_full_size_default_stopping_rule_matches_oracle_fixture():
    """config5's forward: config2 under the reference's default stopping rule
    (tolerance 1e-9, at most 10000 accelerated iterations, early stop;
    kernels.py:228-305).  The oracle leaves samples 0, 511 and 1023 at the
    iteration limit (tests/golden/config2_converged.npz, written by
    tests/golden/make_config2_converged.py); the GPU, on the whole batch, must
    agree on their status, iteration count, residual and iterate.  No sample of
    the batch converges, so none is gradient-eligible (bounds.py:148-153): the
    config5 VJP at this forward is zero by the reference's own rule."""
    require_gpu()
    import os

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                        "config2_converged.npz")
    with np.load(path, allow_pickle=False) as f:
        g = {k: f[k] for k in f.files}
    w = workloads.config2()
    B = w.target.shape[0]
    p, _, _ = full_plan(w)
    rhs = np.tile(w.rhs, (B, 1))
    out = p.project(w.target, rhs, max_iterations=10000, early_stop=True, tolerance=1e-9,
                    shared_bounds=True, save=True)
    s = g["samples"]
    status, iters = to_np(out.status), to_np(out.iterations)
    np.testing.assert_array_equal(status[s], g["status"])
    np.testing.assert_array_equal(iters[s], g["iterations"])
    assert rel_err(to_np(out.y)[s], g["y"]) <= 1e-10
    # the residual is a small difference (~1e-8): relative agreement to 1e-3
    res = to_np(out.residual)[s]
    assert np.all(np.abs(res - g["residual"]) <= 1e-3 * np.abs(g["residual"]))
    assert np.all(status == 1) and int(to_np(out.eligible).sum()) == 0


@pytest.mark.parametrize("edges,dtype", [(12000, np.float64), (9000, np.float64),
                                         (12000, np.float32)])
def test_narrow_column_tiles(edges, dtype):
    """Network flow with 5000 nodes: a wide batch tile's slice of d+ (5000 x 128
    fp64 or x 256 fp32 samples, 5.1 MB) exceeds an XCD's L2, so with 8 narrow
    tiles (B = 256 fp64 / 512 fp32) the fixed-iteration column pass takes a
    quarter wavefront per column.  Checked against the C loop on samples from
    both ends of the batch, and bit-identical to the wide column pass, which a
    batch of 64 / 128 samples runs (samples are independent and both passes
    sum in the same order).  9000 edges (n < 2m) keeps ybar streamed; 12000
    forms K ybar from K y."""
    torch = require_gpu()
    B = 256 if dtype == np.float64 else 512
    w = workloads.config3(batch=B, nodes=5000, edges=edges)
    w.iterations = 200
    w.dtype = np.dtype(dtype)
    w.target = w.target.astype(dtype)
    p, values, root = full_plan(w)
    rhs = np.tile(w.rhs, (B, 1)).astype(dtype)
    for shared in (True, False):
        kw = dict(max_iterations=w.iterations, early_stop=False, shared_bounds=shared)
        print(f"edges={edges} dtype={np.dtype(dtype).name} B={B} shared={shared}", flush=True)
        out = p.project(w.target, rhs, timing=True, **kw)
        t = p.last_timing()
        assert t["resident"] == 0 and t["narrow_columns"] == 1
        assert t["linear_kybar"] == (1 if edges > 2 * 5000 else 0)
        y = to_np(out.y)
        bar = 1e-10 if dtype == np.float64 else 1e-4
        want = checker_y(w, values, root, PICK)
        assert rel_err(y[PICK] * root.astype(dtype), want) <= bar
        k = B // 4
        wide = p.project(w.target[:k], rhs[:k], timing=True, **kw)
        assert p.last_timing()["narrow_columns"] == 0
        np.testing.assert_array_equal(to_np(wide.y), y[:k])
        np.testing.assert_array_equal(to_np(wide.multipliers), to_np(out.multipliers)[:k])
        del out, wide
    torch.cuda.empty_cache()
