"""The reentrant boundary: caller workspaces (``purin_cp_workspace_bytes`` and
the ``workspace`` fields of the options structs).

The reference's layer is pure functional under ``jax.jit``
(src/purin/solvers/chambolle_pock/bounds.py:33, 68-167): XLA owns every
buffer, and one prepared layer may run on several streams at once.  Here a
call given its own workspace allocates nothing and leaves the plan's data
untouched, so calls on one plan may overlap.  Each test compares such calls,
bit for bit, with the same calls made one after another on the plan's own
workspace.  Every call goes through the C ABI.
"""

import threading

import numpy as np
import pytest

from purin_amd import workloads
from purin_amd._lib import ERR_ARG, PurinError
from tests._gpu import canonical_from_workload, plan_for, rel_err, require_gpu, to_np

pytestmark = pytest.mark.gpu

PROJECT_FIELDS = ("y", "multipliers", "slacks", "status", "iterations", "residual", "finite",
                  "eligible")
ADJOINT_FIELDS = ("g_target", "g_rhs", "valid", "info", "residual")


def _same(a, b, fields, what):
    for f in fields:
        x, y = to_np(getattr(a, f)), to_np(getattr(b, f))
        assert x.shape == y.shape, (what, f)
        assert np.array_equal(x, y, equal_nan=True), (what, f, np.max(np.abs(x - y)))


def _problem(batch, n=300, seed=21):
    w = workloads.small_random(seed, n=n, me=n // 7, mi=(2 * n) // 5, width=5, batch=batch,
                               accelerated=True, target_sd=0.5)
    return w, canonical_from_workload(w)


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
def test_caller_workspace_matches_the_plans_own(dtype):
    """project (resident fixed and early stop, streaming early stop), solve and
    adjoint with a workspace of exactly the queried size give the plan-workspace
    bits, and leave the plan's own workspaces unallocated."""
    torch = require_gpu()
    B = 64
    w, canon = _problem(B)
    plan = plan_for(canon, dtype=dtype, accelerated=True)
    target = torch.as_tensor(w.target.astype(dtype), device="cuda")
    rhs = torch.as_tensor(np.tile(w.rhs, (B, 1)).astype(dtype), device="cuda")
    modes = {"fixed": dict(early_stop=False), "early": dict(early_stop=True),
             "streaming": dict(early_stop=True, streaming=True)}
    got = {}
    for name, kw in modes.items():
        print(f"caller workspace: project {name} {np.dtype(dtype).name}", flush=True)
        ws = plan.new_workspace("project", B)
        got[name] = plan.project(target, rhs, max_iterations=500, tolerance=1e-3, save=True,
                                 workspace=ws, **kw)
    cot = torch.as_tensor(np.random.default_rng(3).normal(size=(B, w.n)).astype(dtype),
                          device="cuda")
    wsa = plan.new_workspace("adjoint", B)
    adj = plan.adjoint(got["fixed"].saved, None, None, cot, force_eligible=True, workspace=wsa,
                       return_steps=True)
    torch.cuda.synchronize()
    info = plan.current_info()
    assert info.workspace_bytes == 0 and info.adjoint_workspace_bytes == 0
    # the same calls on the plan's own workspace
    for name, kw in modes.items():
        want = plan.project(target, rhs, max_iterations=500, tolerance=1e-3, save=True, **kw)
        _same(got[name], want, PROJECT_FIELDS, name)
        if name == "fixed":
            saved_plan = want.saved
    assert np.any(to_np(got["early"].iterations) < 500)  # the stop test fired
    want_adj = plan.adjoint(saved_plan, None, None, cot, force_eligible=True)
    _same(adj, want_adj, ADJOINT_FIELDS, "adjoint")
    np.testing.assert_array_equal(to_np(adj.steps), to_np(plan.last_adjoint_iterations(B)))
    assert plan.current_info().workspace_bytes > 0
    # solve with its own workspace
    pre_rhs = torch.as_tensor(np.zeros((B, plan.m), dtype), device="cuda")
    lo = torch.full((B, w.n), -1.0, dtype=target.dtype, device="cuda")
    hi = torch.full((B, w.n), 1.0, dtype=target.dtype, device="cuda")
    s1 = plan.solve(pre_rhs, target, lo, hi, max_iterations=300, early_stop=False,
                    workspace=plan.new_workspace("solve", B))
    s2 = plan.solve(pre_rhs, target, lo, hi, max_iterations=300, early_stop=False)
    _same(s1, s2, ("y", "dual", "iterations", "residual", "gap", "converged"), "solve")


def test_workspace_too_small_or_misaligned_is_an_argument_error():
    torch = require_gpu()
    B = 16
    w, canon = _problem(B)
    plan = plan_for(canon, dtype=np.float64, accelerated=True)
    rhs = np.tile(w.rhs, (B, 1))
    need = plan.workspace_bytes("project", B)
    assert need > 0
    assert plan.workspace_bytes("project", 20 * B) > need  # 16 and 320 pad to 128 and 384
    assert plan.workspace_bytes("adjoint", B, restart=10) < plan.workspace_bytes("adjoint", B)
    ws = torch.empty(need + 512, dtype=torch.uint8, device="cuda")
    # (the query is the largest over the optional arguments: this call, with no
    # warm start, needs less, so cut well below it)
    with pytest.raises(PurinError) as err:
        plan.project(w.target, rhs, max_iterations=10, workspace=ws[:need // 4])
    assert err.value.code == ERR_ARG and "too small" in str(err.value)
    with pytest.raises(PurinError) as err:
        plan.project(w.target, rhs, max_iterations=10, workspace=ws[8:need + 8])
    assert err.value.code == ERR_ARG and "aligned" in str(err.value)
    with pytest.raises(PurinError):
        plan.workspace_bytes("project", 0)
    out = plan.project(w.target, rhs, max_iterations=10, workspace=ws[:need])
    torch.cuda.synchronize()
    assert np.all(np.isfinite(to_np(out.y)))


def test_two_streams_on_one_plan():
    """Two projections of different inputs on one plan, launched on two streams
    without any ordering between them, each with its own workspace: the same
    bits as the two calls made one after the other."""
    torch = require_gpu()
    B = 256
    w, canon = _problem(B, n=700)
    plan = plan_for(canon, dtype=np.float64, accelerated=True)
    rng = np.random.default_rng(8)
    ta = torch.as_tensor(w.target, device="cuda")
    tb = torch.as_tensor(w.target + rng.normal(scale=0.3, size=w.target.shape), device="cuda")
    rhs = torch.as_tensor(np.tile(w.rhs, (B, 1)), device="cuda")
    kw = dict(max_iterations=1500, early_stop=False, save=True)
    want_a = plan.project(ta, rhs, **kw)
    want_b = plan.project(tb, rhs, **kw)
    wsa, wsb = plan.new_workspace("project", B), plan.new_workspace("project", B)
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    main = torch.cuda.current_stream()
    sa.wait_stream(main)
    sb.wait_stream(main)
    print("two streams: launching", flush=True)
    with torch.cuda.stream(sa):
        got_a = plan.project(ta, rhs, workspace=wsa, **kw)
    with torch.cuda.stream(sb):
        got_b = plan.project(tb, rhs, workspace=wsb, **kw)
    torch.cuda.synchronize()
    _same(got_a, want_a, PROJECT_FIELDS, "stream a")
    _same(got_b, want_b, PROJECT_FIELDS, "stream b")
    assert not np.array_equal(to_np(got_a.y), to_np(got_b.y))


def test_two_threads_on_one_plan():
    """Two host threads, each with its own stream and workspaces, run an
    early-stop projection on the streaming passes (which read the device's
    all-done flag through the plan's pinned slots) and then the adjoint (which
    reads its per-step counts the same way) on one plan at the same time."""
    torch = require_gpu()
    B = 96
    w, canon = _problem(B, n=400, seed=5)
    plan = plan_for(canon, dtype=np.float64, accelerated=True)
    rng = np.random.default_rng(2)
    targets = [torch.as_tensor(w.target + rng.normal(scale=0.2, size=w.target.shape),
                               device="cuda") for _ in range(2)]
    cots = [torch.as_tensor(rng.normal(size=(B, w.n)), device="cuda") for _ in range(2)]
    rhs = torch.as_tensor(np.tile(w.rhs, (B, 1)), device="cuda")
    kw = dict(max_iterations=1200, early_stop=True, tolerance=1e-4, streaming=True,
              check_every=5, save=True)
    want = []
    for t, c in zip(targets, cots):
        f = plan.project(t, rhs, **kw)
        a = plan.adjoint(f.saved, None, None, c, force_eligible=True)
        want.append((f, a, to_np(plan.last_adjoint_iterations(B))))
    torch.cuda.synchronize()
    got, errors = [None, None], []

    def work(k):
        try:
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.default_stream())
            with torch.cuda.stream(s):
                f = plan.project(targets[k], rhs, workspace=plan.new_workspace("project", B),
                                 **kw)
                a = plan.adjoint(f.saved, None, None, cots[k], force_eligible=True,
                                 workspace=plan.new_workspace("adjoint", B), return_steps=True)
            s.synchronize()
            got[k] = (f, a)
        except Exception as e:  # reported by the main thread
            errors.append(e)

    print("two threads: starting", flush=True)
    threads = [threading.Thread(target=work, args=(k,)) for k in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a thread did not finish"
    assert not errors, errors
    for k in range(2):
        f, a = got[k]
        _same(f, want[k][0], PROJECT_FIELDS, ("thread project", k))
        _same(a, want[k][1], ADJOINT_FIELDS, ("thread adjoint", k))
        np.testing.assert_array_equal(to_np(a.steps), want[k][2])
        assert np.any(to_np(f.iterations) < kw["max_iterations"])


def test_schedule_extension_beyond_65536_iterations():
    """The resident kernel reads a step schedule built for 65536 iterations; a
    longer call extends it once (uploaded on the plan's own stream).  Two
    threads extend it at once (70000 and 90000 iterations), then a third call
    (100000) reads the extended schedule: each against the streaming passes,
    whose host loop computes the same accelerated steps, at the fp64 bar."""
    torch = require_gpu()
    B = 32
    w, canon = _problem(B, n=48, seed=12)
    plan = plan_for(canon, dtype=np.float64, accelerated=True)
    rhs = torch.as_tensor(np.tile(w.rhs, (B, 1)), device="cuda")
    target = torch.as_tensor(w.target, device="cuda")
    results, errors = {}, []

    def run(iters):
        try:
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.default_stream())
            with torch.cuda.stream(s):
                r = plan.project(target, rhs, max_iterations=iters, early_stop=False,
                                 workspace=plan.new_workspace("project", B))
            s.synchronize()
            results[iters] = r
        except Exception as e:
            errors.append(e)

    print("schedule extension: two threads", flush=True)
    threads = [threading.Thread(target=run, args=(k,)) for k in (70000, 90000)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=300)
    assert not any(t.is_alive() for t in threads) and not errors, errors
    print("schedule extension: 100000 iterations", flush=True)
    results[100000] = plan.project(target, rhs, max_iterations=100000, early_stop=False,
                                   timing=True)
    assert plan.last_timing()["resident"] == 1
    for iters, got in results.items():
        want = plan.project(target, rhs, max_iterations=iters, early_stop=False, streaming=True)
        torch.cuda.synchronize()
        assert rel_err(to_np(got.y), to_np(want.y)) <= 1e-10, iters
        np.testing.assert_array_equal(to_np(got.iterations), iters)
