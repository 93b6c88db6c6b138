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


def checker_y(w, values, root, samples):
    """y of the C loop for ``samples`` (in the metric's variables when there is one)."""
    rows = [list(w.indices[w.indptr[i]:w.indptr[i + 1]]) for i in range(w.rows_total)]
    coef = [list(values[w.indptr[i]:w.indptr[i + 1]]) for i in range(w.rows_total)]
    canon = op.Canonical(n=w.n, me=w.me, rows=rows, coef=coef)
    target = np.asarray(w.target[samples], w.dtype)
    if root is not None:
        target = target * root.astype(w.dtype)
    rhs = np.tile(w.rhs, (len(samples), 1)).astype(w.dtype)
    cfg = op.Config(accelerated=w.accelerated, max_iterations=w.iterations, early_stop=False)
    y, _, _ = cloop.run(cloop.prepare(canon, target, rhs, cfg, w.dtype), w.iterations,
                        w.accelerated, threads=4)
    return y


@pytest.mark.parametrize("config", [2, 3, 4])
def test_full_size_projection(config):
    torch = require_gpu()
    w = {2: workloads.config2, 3: workloads.config3, 4: workloads.config4}[config]()
    B = w.target.shape[0]
    p, values, root = full_plan(w)
    rhs = np.tile(w.rhs, (B, 1)).astype(w.dtype)
    kw = dict(max_iterations=w.iterations, early_stop=False, shared_bounds=True)
    print(f"config{config}: B={B} n={w.n} iterations={w.iterations}", flush=True)
    out = p.project(w.target, rhs, **kw)
    y = to_np(out.y)
    bar = 1e-10 if w.dtype == np.float64 else 1e-4
    want = checker_y(w, values, root, PICK)
    got = y[PICK] * (root if root is not None else 1.0)
    assert rel_err(got, want) <= bar
    # independence of samples: the leading half alone is bit-identical
    k = B // 2
    alone = p.project(w.target[:k], rhs[:k], **kw)
    np.testing.assert_array_equal(to_np(alone.y), y[:k])
    np.testing.assert_array_equal(to_np(alone.status), to_np(out.status)[:k])
    np.testing.assert_array_equal(to_np(alone.multipliers), to_np(out.multipliers)[:k])
    del out, alone
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


def test_full_size_adjoint_at_the_same_state():
    """config5: the VJP of the full 1024-sample batch (eligibility forced at the
    2000-iteration state, default GMRES) against the oracle's adjoint on a few
    samples linearised at the GPU's own state."""
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
    adj = p.adjoint(saved, w.target, rhs_k, w.cotangent, force_eligible=True, rhs_rows=p.m)
    info = to_np(adj.info)
    ksup, kmask = pre.support[pre.rows], pre.mask[pre.rows]
    sub = PICK[[0, -1]]
    want = oadj.adjoint(pre.kept_values[0], ksup, kmask, w.me, to_np(o.y)[sub], to_np(o.dual)[sub],
                        np.ones(len(sub), bool), w.target[sub], rhs_k[sub],
                        np.broadcast_to(pre.lower[0], (len(sub), w.n)),
                        np.broadcast_to(pre.upper[0], (len(sub), w.n)), w.cotangent[sub], cfg)
    np.testing.assert_array_equal(info[sub], want.info)
    assert rel_err(to_np(adj.g_target)[sub], want.g_target) <= 1e-8
    assert rel_err(to_np(adj.g_rhs)[sub], want.g_rhs) <= 1e-8
