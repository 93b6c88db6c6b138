"""The no-allocation projection entry (``purin_cp_project_noalloc``) against
``purin_cp_project``: the same kernels on the same inputs, so every output must
be identical bit for bit.  Both are called through the C ABI (ctypes).

Two calls in a row on each path, the second with a smaller batch (and other
inputs), so the scratch array's leftover contents from the first call must not
leak into the second.
"""

import numpy as np
import pytest

from purin_amd import workloads
from tests._gpu import canonical_from_workload, plan_for, require_gpu, to_np

pytestmark = pytest.mark.gpu

FIELDS = ("y", "multipliers", "slacks", "status", "iterations", "residual", "finite", "eligible")


def _same(a, b, what):
    for f in FIELDS:
        x, y = to_np(getattr(a, f)), to_np(getattr(b, f))
        assert x.shape == y.shape, (what, f)
        assert np.array_equal(x, y, equal_nan=True), (what, f, np.max(np.abs(x - y)))


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("mode", ["fixed", "early", "streaming", "shared_bounds"])
def test_noalloc_matches_project_on_two_calls(dtype, mode):
    torch = require_gpu()
    w = workloads.small_random(21, n=300, me=40, mi=120, width=5, batch=96, accelerated=True,
                               target_sd=0.5)
    canon = canonical_from_workload(w)
    plan = plan_for(canon, dtype=dtype, accelerated=True)
    rng = np.random.default_rng(4)
    kw = dict(max_iterations=600, tolerance=1e-3,
              early_stop=mode in ("early", "shared_bounds"), streaming=mode == "streaming",
              shared_bounds=mode == "shared_bounds")
    for batch in (96, 37):  # the second call is smaller
        print(f"noalloc {mode} {np.dtype(dtype).name} batch {batch}", flush=True)
        target = (w.target[:batch] + rng.normal(scale=0.05, size=(batch, w.n))).astype(dtype)
        rhs = np.tile(w.rhs, (batch, 1)).astype(dtype)
        want = plan.project(target, rhs, **kw)
        got = plan.project(target, rhs, noalloc=True, **kw)
        torch.cuda.synchronize()
        _same(got, want, (mode, batch))
        if kw["early_stop"]:  # the stop test fired, so the frozen samples are covered
            assert np.any(to_np(want.iterations) < kw["max_iterations"])


def test_noalloc_config2_shape_and_warm_start():
    """The headline shape (n = 4096, 1024 + 2048 kept rows, 8192 bound rows) at
    the largest batch the scratch holds, with warm-start multipliers, then a
    smaller call."""
    torch = require_gpu()
    w = workloads.config2(batch=128)
    canon = canonical_from_workload(w)
    plan = plan_for(canon, dtype=np.float64, accelerated=True)
    rng = np.random.default_rng(9)
    for batch in (128, 50):
        print(f"noalloc config2 batch {batch}", flush=True)
        target = w.target[:batch]
        rhs = np.tile(w.rhs, (batch, 1))
        mult0 = np.abs(rng.normal(size=(batch, canon.me + canon.mi))) * 0.01
        kw = dict(max_iterations=200, early_stop=False, multipliers0=mult0)
        want = plan.project(target, rhs, **kw)
        got = plan.project(target, rhs, noalloc=True, **kw)
        torch.cuda.synchronize()
        _same(got, want, ("config2", batch))


def test_noalloc_rejects_what_does_not_fit():
    torch = require_gpu()
    from purin_amd._lib import ERR_ARG, PurinError

    w = workloads.config2(batch=1024)
    canon = canonical_from_workload(w)
    plan = plan_for(canon, dtype=np.float64, accelerated=True)
    rhs = np.tile(w.rhs, (1024, 1))
    with pytest.raises(PurinError) as err:
        plan.project(w.target, rhs, max_iterations=10, early_stop=False, noalloc=True)
    assert err.value.code == ERR_ARG and "scratch" in str(err.value)
    small = w.target[:8]
    with pytest.raises(PurinError) as err:
        plan.project(small, rhs[:8], max_iterations=(1 << 16) + 1, early_stop=False,
                     noalloc=True)
    assert err.value.code == ERR_ARG and "schedule" in str(err.value)
    with pytest.raises(PurinError) as err:
        plan.project(small, rhs[:8], max_iterations=10, timing=True, noalloc=True)
    assert err.value.code == ERR_ARG
    # the regular entry still runs afterwards
    out = plan.project(small, rhs[:8], max_iterations=10, early_stop=False)
    torch.cuda.synchronize()
    assert np.all(np.isfinite(to_np(out.y)))


def test_noalloc_allocates_nothing():
    """On a fresh plan the no-allocation entry leaves the plan's workspace
    unallocated, and after a regular call has sized it, a no-allocation call with
    a larger batch leaves its size unchanged (purin_cp_plan_info.workspace_bytes)."""
    torch = require_gpu()
    w = workloads.small_random(23, n=300, me=40, mi=120, width=5, batch=96, accelerated=True,
                               target_sd=0.5)
    canon = canonical_from_workload(w)
    plan = plan_for(canon, dtype=np.float64, accelerated=True)
    rhs = np.tile(w.rhs, (96, 1))
    for mode in ({}, dict(early_stop=True), dict(early_stop=True, streaming=True)):
        kw = dict(max_iterations=300, tolerance=1e-3, early_stop=False)
        kw.update(mode)
        plan.project(w.target, rhs, noalloc=True, **kw)
    torch.cuda.synchronize()
    assert plan.current_info().workspace_bytes == 0
    small = plan.project(w.target[:16], rhs[:16], max_iterations=300, early_stop=False)
    torch.cuda.synchronize()
    sized = plan.current_info().workspace_bytes
    assert sized > 0
    big = plan.project(w.target, rhs, max_iterations=300, early_stop=False, noalloc=True)
    torch.cuda.synchronize()
    assert plan.current_info().workspace_bytes == sized
    np.testing.assert_array_equal(to_np(big.y)[:16], to_np(small.y))


def test_noalloc_under_graph_capture():
    """A fixed-iteration no-allocation projection captured into a graph and
    replayed three times on new inputs (with eager calls and synchronisations
    between the replays) gives the bits of purin_cp_project on each input.  An
    early-stop call on the streaming passes, which would read a device flag, is
    refused under capture before it enqueues anything."""
    torch = require_gpu()
    B = 64
    w = workloads.small_random(24, n=300, me=40, mi=120, width=5, batch=B, accelerated=True,
                               target_sd=0.5)
    canon = canonical_from_workload(w)
    plan = plan_for(canon, dtype=np.float64, accelerated=True)
    rng = np.random.default_rng(6)
    target = torch.as_tensor(w.target, device="cuda")
    rhs = torch.as_tensor(np.tile(w.rhs, (B, 1)), device="cuda")
    kw = dict(max_iterations=400, early_stop=False)
    plan.project(target, rhs, noalloc=True, **kw)  # warm-up outside the capture
    torch.cuda.synchronize()
    print("graph capture: capturing", flush=True)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, capture_error_mode="relaxed"):
        out = plan.project(target, rhs, noalloc=True, **kw)
    torch.cuda.synchronize()
    for k in range(3):
        new_t = w.target + rng.normal(scale=0.2, size=w.target.shape)
        target.copy_(torch.as_tensor(new_t, device="cuda"))
        torch.cuda.synchronize()
        print(f"graph capture: replay {k}", flush=True)
        g.replay()
        torch.cuda.synchronize()
        want = plan.project(torch.as_tensor(new_t, device="cuda"), rhs, **kw)
        torch.cuda.synchronize()
        _same(out, want, ("replay", k))
    # refused before anything is enqueued
    g2 = torch.cuda.CUDAGraph()
    side = torch.zeros(4, device="cuda")
    from purin_amd._lib import ERR_ARG, PurinError

    with pytest.raises(PurinError) as err:
        with torch.cuda.graph(g2, capture_error_mode="relaxed"):
            side.add_(1.0)
            plan.project(target, rhs, noalloc=True, max_iterations=50, early_stop=True,
                         streaming=True)
    assert err.value.code == ERR_ARG and "capture" in str(err.value)
    torch.cuda.synchronize()
