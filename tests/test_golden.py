"""The committed config1 fixture (tests/golden/config1.npz) is what the oracle computes.

CPU only.  Guards the fixture (and the oracle) against drift; the GPU tests in
tests/test_gpu_golden.py compare the HIP path with the same fixture.
"""

import numpy as np

from oracle import projection as op
from purin_amd import workloads
from tests import _golden


def test_fixture_inputs_are_the_config1_generator():
    g = _golden.load()
    w = workloads.config1(batch=32)
    np.testing.assert_array_equal(g["indptr"], w.indptr)
    np.testing.assert_array_equal(g["indices"], w.indices)
    np.testing.assert_array_equal(g["data"], w.data)
    np.testing.assert_array_equal(g["rhs"], w.rhs)
    np.testing.assert_array_equal(g["target"], w.target)
    np.testing.assert_array_equal(g["cot"], np.random.default_rng(5).normal(0.0, 1.0, (32, 64)))


def test_oracle_reproduces_fixed_iteration_outputs():
    g = _golden.load()
    canon = _golden.canonical(g)
    rhs = np.tile(g["rhs"], (32, 1))
    for tag, dtype, tol in (("f64", np.float64, 1e-12), ("f32", np.float32, 1e-5)):
        cfg = op.Config(accelerated=False, max_iterations=1000, early_stop=False)
        r = op.solve(canon, g["target"].astype(dtype), rhs.astype(dtype), cfg, dtype=dtype)
        mult = np.concatenate((r.multipliers_eq, r.multipliers_ineq), axis=1)
        for got, name in ((r.y, "y"), (mult, "multipliers"), (r.slacks, "slacks")):
            want = g[f"{tag}_{name}"]
            assert np.max(np.abs(got - want)) <= tol * max(1.0, np.max(np.abs(want))), name
        np.testing.assert_array_equal(r.status, g[f"{tag}_status"])
        np.testing.assert_array_equal(r.iterations, g[f"{tag}_iterations"])


def test_oracle_reproduces_converged_vjp():
    g = _golden.load()
    canon = _golden.canonical(g)
    rhs = np.tile(g["rhs"], (32, 1))
    cfg = op.Config(accelerated=False, max_iterations=10000, tolerance=1e-9)
    res, g_target, g_rhs, adj = op.vjp(canon, g["target"], rhs, cfg, g["cot"])
    np.testing.assert_array_equal(res.status, g["conv_status"])
    np.testing.assert_array_equal(res.iterations, g["conv_iterations"])
    np.testing.assert_allclose(res.y, g["conv_y"], rtol=0, atol=1e-12)
    np.testing.assert_allclose(g_target, g["conv_g_target"], rtol=0, atol=1e-10)
    np.testing.assert_allclose(g_rhs, g["conv_g_rhs"], rtol=0, atol=1e-10)
