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
