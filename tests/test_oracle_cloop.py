"""The C restatement of the fixed-iteration CP loop (oracle/cp_loop.c) equals the
NumPy oracle bit for bit (same operation order, no FMA contraction).

CPU only.  The C loop is the CPU baseline ``bench.py`` times; this pins it.
"""

import numpy as np
import pytest

from oracle import cloop
from oracle import projection as op
from purin_amd import workloads


@pytest.fixture(scope="module", autouse=True)
def built():
    cloop.build()


def canonical(w):
    return op.Canonical(n=w.n, me=w.me, rows=w.rows(), coef=w.coefs())


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("case", ["config1", "accelerated", "warm"])
def test_c_loop_equals_numpy_oracle(dtype, case):
    if case == "config1":
        w = workloads.config1()
    else:
        w = workloads.small_random(11, n=300, me=30, mi=90, width=6, batch=9, accelerated=True)
    canon = canonical(w)
    B = w.target.shape[0]
    rhs = np.tile(w.rhs, (B, 1)).astype(dtype)
    target = w.target.astype(dtype)
    rng = np.random.default_rng(3)
    mult = None
    if case == "warm":
        mult = np.abs(rng.normal(size=(B, w.rows_total))).astype(dtype)
    cfg = op.Config(accelerated=w.accelerated, max_iterations=250, early_stop=False)
    _, out, pre = op.solve(canon, target, rhs, cfg, dtype=dtype, return_internal=True,
                           multipliers_eq=None if mult is None else mult[:, :w.me],
                           multipliers_ineq=None if mult is None else mult[:, w.me:])
    prep = cloop.prepare(canon, target, rhs, cfg, dtype)
    dual0 = None if mult is None else (mult[:, pre.rows] / pre.scale).astype(dtype)
    for threads in (1, 3):
        y, d, _ = cloop.run(prep, 250, w.accelerated, threads=threads, dual0=dual0)
        np.testing.assert_array_equal(y, out.y)
        np.testing.assert_array_equal(d, out.dual)


def test_c_loop_propagates_nan_like_the_oracle():
    w = workloads.config1(batch=4)
    canon = canonical(w)
    target = w.target.copy()
    target[1, 3] = np.nan
    rhs = np.tile(w.rhs, (4, 1))
    cfg = op.Config(accelerated=False, max_iterations=20, early_stop=False)
    _, out, _ = op.solve(canon, target, rhs, cfg, return_internal=True)
    y, d, _ = cloop.run(cloop.prepare(canon, target, rhs, cfg), 20, False)
    np.testing.assert_array_equal(np.isnan(y), np.isnan(out.y))
    np.testing.assert_array_equal(np.isnan(d), np.isnan(out.dual))
    ok = ~np.isnan(out.y)
    np.testing.assert_array_equal(y[ok], out.y[ok])
